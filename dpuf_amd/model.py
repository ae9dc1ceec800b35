"""Python host helpers around libdpuf_tools.so: build or open a model (mode 12,
or the mode 13 / 14 had4p-hybrid plan with weight_plan=1)
and hand its C descriptors to an engine.  Mirrors the role of the reference's
Python host (dpuf_format.py:2130-2357), with the token loop on the GPU.
"""
import ctypes as C

import numpy as np

from . import abi

# Model shapes used by the workloads (hidden, inter, layers, q heads, kv heads,
# head_dim, vocab).  Qwen3-0.6B and Qwen3-8B shapes.
QWEN3_0_6B = dict(hidden_size=1024, intermediate_size=3072, num_layers=28, num_q_heads=16,
                  num_kv_heads=8, head_dim=128, vocab_size=151936, tie_word_embeddings=1)
QWEN3_8B = dict(hidden_size=4096, intermediate_size=12288, num_layers=36, num_q_heads=32,
                num_kv_heads=8, head_dim=128, vocab_size=151936, tie_word_embeddings=0)


def make_spec(shape, max_seq_len=128, seed=1234, std=0.02, **over):
    d = dict(shape)
    d.update(over)
    s = abi.DpufToolsSpec()
    for k, v in d.items():
        setattr(s, k, v)
    s.max_seq_len = max_seq_len
    s.weight_std = std
    s.rms_eps = 1e-6
    s.rope_theta = 1e6
    s.seed = seed
    return s


class Model:
    """Owns a DpufToolsModel (built in memory or mmapped from a .dpuf)."""

    def __init__(self, handle):
        if not handle:
            raise RuntimeError("model build/open failed")
        self.lib = abi.load_tools()
        self.h = handle

    @classmethod
    def build(cls, shape, **kw):
        lib = abi.load_tools()
        spec = make_spec(shape, **kw)
        return cls(lib.dpuf_tools_build_model(C.byref(spec)))

    @classmethod
    def open(cls, path, verify=False, max_seq_len=0):
        lib = abi.load_tools()
        st = C.c_int32(0)
        h = lib.dpuf_tools_open_container(path.encode(), int(verify), int(max_seq_len), C.byref(st))
        if not h:
            raise RuntimeError(f"open_container failed with status {st.value}")
        return cls(h)

    def save(self, path):
        return self.lib.dpuf_tools_save_container(self.h, path.encode())

    @property
    def cfg(self):
        return self.lib.dpuf_tools_model_cfg(self.h)

    @property
    def layers(self):
        return self.lib.dpuf_tools_model_layers(self.h)

    @property
    def tok(self):
        return self.lib.dpuf_tools_model_tok(self.h)

    @property
    def lm(self):
        return self.lib.dpuf_tools_model_lm(self.h)

    @property
    def out_norm(self):
        return self.lib.dpuf_tools_model_out_norm(self.h)

    @property
    def healed(self):
        return self.lib.dpuf_tools_model_healed(self.h)

    def weight_bytes(self):
        return int(self.lib.dpuf_tools_model_weight_bytes(self.h))

    def create_args(self, cfg=None):
        """Arguments of dpuf_engine_create / orc_engine_create."""
        c = cfg if cfg is not None else self.cfg.contents
        return (C.byref(c), self.layers, self.tok, self.lm, self.out_norm)

    def close(self):
        if self.h:
            self.lib.dpuf_tools_free_model(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def desc_tile_bytes(d):
    """Total tile bytes (tile_offsets[n_tiles]) of a DpufWeightDesc."""
    offs = C.cast(d.tile_offsets, C.POINTER(C.c_uint64))
    return int(offs[d.n_tiles])


def ptr(a):
    """ctypes void pointer of a contiguous numpy array (None for None)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


def pack_matrix(W, sign_bits, ecc_group=64, mode=12, w_pow=0.0):
    """Packs an fp32 [rows, cols] array into a mode 12, 13 or 14 blob
    (bytes-like ndarray) and returns (blob, desc).  The blob must outlive the
    desc."""
    lib = abi.load_tools()
    W = np.ascontiguousarray(W, dtype=np.float32)
    sb = np.ascontiguousarray(sign_bits, dtype=np.uint8)
    n = C.c_size_t(0)
    if mode == 12:
        p = lib.dpuf_tools_pack_mode12(ptr(W), W.shape[0], W.shape[1], ptr(sb), ecc_group, C.byref(n))
    else:
        p = lib.dpuf_tools_pack_asym(ptr(W), W.shape[0], W.shape[1], ptr(sb), ecc_group, 4 if mode == 13 else 6,
                                     w_pow, C.byref(n))
    if not p:
        raise RuntimeError("pack failed")
    blob = np.frombuffer((C.c_uint8 * n.value).from_address(p), dtype=np.uint8).copy()
    lib._free(p)
    d = abi.DpufWeightDesc()
    assert lib.dpuf_tools_bind_blob(ptr(blob), blob.size, C.byref(d)) == 0
    return blob, d


def random_normal(n, std, seed, name):
    lib = abi.load_tools()
    out = np.empty(n, dtype=np.float32)
    lib.dpuf_tools_random_normal(ptr(out), n, std, seed, name.encode())
    return out


def sign_bits(cols, seed, name):
    lib = abi.load_tools()
    out = np.empty(cols // 8, dtype=np.uint8)
    lib.dpuf_tools_sign_bits(ptr(out), cols, seed, name.encode())
    return out


def desc_arrays(d):
    """(tiles uint8 view, tile_offsets uint64 view, sign bits) of a desc."""
    offs = np.ctypeslib.as_array(C.cast(d.tile_offsets, C.POINTER(C.c_uint64)), shape=(d.n_tiles + 1,))
    tiles = np.ctypeslib.as_array(C.cast(d.tensor_base, C.POINTER(C.c_uint8)), shape=(int(offs[-1]),))
    sb = np.ctypeslib.as_array(C.cast(d.sign_bits, C.POINTER(C.c_uint8)), shape=(d.cols // 8,))
    return tiles, offs, sb
