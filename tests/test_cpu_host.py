"""Host-side checks that need no GPU: the C-ABI library loads and exports
every declared symbol with the reference struct layouts, argument errors are
reported without touching a device, and the .dpuf ingest path (container
writer/reader, tile CRC32 verify, XOR-parity heal) behaves like the
reference CLI's (dpuf-cli.c:1669-1731, dpuf_avx2.c:846-908)."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from dpuf_amd import abi
from dpuf_amd import model as M

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

TINY = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)


def declared_exports():
    names = []
    for h in ("dpuf_kernels.h", "dpuf_amd.h"):
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"DPUF_EXPORT\s+[\w\s\*]+?\b(\w+)\s*\(", text):
            names.append(m.group(1))
    return names


def test_library_exports_every_declared_symbol():
    names = declared_exports()
    assert len(names) >= 30
    lib = C.CDLL(abi.lib_path("libdpuf_amd.so"))
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    for n in abi.ENGINE_SYMBOLS:
        assert n in names


def test_struct_layouts_match_reference(tmp_path):
    """DpufWeightDesc 48 B, DpufModelConfig 92 B, DpufLayerWeights 368 B
    (reference dpuf_kernels.h:44-101), checked with the C compiler too."""
    assert C.sizeof(abi.DpufWeightDesc) == 48
    assert C.sizeof(abi.DpufModelConfig) == 92
    assert C.sizeof(abi.DpufLayerWeights) == 368
    src = r'''
#include <stddef.h>
#include <stdio.h>
#include "dpuf_kernels.h"
int main(void) {
  printf("%zu %zu %zu %zu %zu %zu %zu %zu\n", sizeof(DpufWeightDesc), sizeof(DpufModelConfig),
         sizeof(DpufLayerWeights), sizeof(DpufQrTileHdr), offsetof(DpufWeightDesc, sign_bits),
         offsetof(DpufModelConfig, kv_type), offsetof(DpufLayerWeights, w_down),
         offsetof(DpufModelConfig, mrope_interleaved));
  return 0;
}
'''
    tmp = str(tmp_path / "layout_check")
    with open(tmp + ".c", "w") as f:
        f.write(src)
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), tmp + ".c", "-o", tmp], check=True)
    out = subprocess.run([tmp], capture_output=True, text=True, check=True).stdout.split()
    assert [int(v) for v in out] == [48, 92, 368, 16, 40, 68, 320, 88]
    assert abi.DpufModelConfig.kv_type.offset == 68
    assert abi.DpufLayerWeights.w_down.offset == 320


def test_engine_argument_errors_without_a_device():
    eng = abi.load_engine()
    ids = np.zeros(4, np.int32)
    lg = np.zeros(16, np.float32)
    assert eng.dpuf_engine_forward_batch(None, 4, M.ptr(ids), 0, 1, M.ptr(lg)) == -1
    assert eng.dpuf_engine_forward_token(None, 1, 0, M.ptr(lg)) == -1
    assert eng.dpuf_engine_forward_batch_ex(None, 4, M.ptr(ids), 0, None, None, None, None, None, 1, M.ptr(lg)) == -1
    assert eng.dpuf_engine_set_slot(None, 0) == -1
    assert eng.dpuf_engine_num_slots(None) == 1
    assert eng.dpuf_engine_get_prefix_len(None, 0) == 0
    assert eng.dpuf_engine_freeze_prefix(None, 0, 4) == 0
    assert eng.dpuf_engine_apply_prefix(None, 0, 0) == 0
    eng.dpuf_engine_destroy(None)
    eng.dpuf_engine_reset_cache(None)


def test_engine_refuses_to_run_without_hip_device():
    """No CPU fallback: without a visible HIP device create returns NULL."""
    eng = abi.load_engine()
    if eng.dpuf_amd_device_ok():
        pytest.skip("a HIP device is visible")
    m = M.Model.build(TINY, max_seq_len=32, seed=3)
    assert not eng.dpuf_engine_create(*m.create_args())


def test_crc32_known_answer(tools):
    data = np.frombuffer(b"123456789", np.uint8).copy()
    assert tools.dpuf_crc32_bytes(M.ptr(data), 9) == 0xCBF43926
    eng = abi.load_engine()
    assert eng.dpuf_crc32_bytes(M.ptr(data), 9) == 0xCBF43926
    assert tools.dpuf_crc32_bytes(M.ptr(data), 0) == 0


def test_container_roundtrip_and_heal(tmp_path, tools):
    m = M.Model.build(TINY, max_seq_len=32, seed=21)
    path = str(tmp_path / "tiny.dpuf")
    n = m.save(path)
    assert n > 0 and os.path.getsize(path) == n
    r = M.Model.open(path, verify=True)
    assert r.healed == 0
    assert r.weight_bytes() == m.weight_bytes()
    for a, b in ((m.tok.contents, r.tok.contents), (m.layers[1].w_down, r.layers[1].w_down)):
        ta, oa, sa = M.desc_arrays(a)
        tb, ob, sb = M.desc_arrays(b)
        assert np.array_equal(ta, tb) and np.array_equal(oa, ob) and np.array_equal(sa, sb)
    cfg = r.cfg.contents
    assert (cfg.hidden_size, cfg.num_layers, cfg.vocab_size, cfg.head_dim) == (256, 2, 4096, 64)
    r.close()

    # locate the tiles of one tensor and corrupt one byte of tile 3
    d = m.layers[0].w_gate
    tiles, offs, _ = M.desc_arrays(d)
    raw = np.fromfile(path, np.uint8)
    needle = tiles[int(offs[3]):int(offs[3]) + 64].tobytes()
    at = raw.tobytes().find(needle)
    assert at > 0
    bad = raw.copy()
    bad[at + 40] ^= 0x5A
    p1 = str(tmp_path / "one_bad.dpuf")
    bad.tofile(p1)
    h = M.Model.open(p1, verify=True)
    assert h.healed == 1
    t2, o2, _ = M.desc_arrays(h.layers[0].w_gate)
    assert np.array_equal(t2, tiles)  # healed copy equals the original tiles
    h.close()
    ok = np.zeros(d.n_tiles, np.uint8)
    hb = bad[at - int(offs[3]):].copy()
    nbad = tools.dpuf_qr_verify_tiles_ex(12, d.n_tiles, d.cols, M.ptr(hb), d.tile_offsets, M.ptr(ok))
    assert nbad == 1 and ok[3] == 0 and ok.sum() == d.n_tiles - 1

    # two bad tiles in the same ECC group cannot be healed
    bad2 = bad.copy()
    at4 = raw.tobytes().find(tiles[int(offs[4]):int(offs[4]) + 64].tobytes())
    bad2[at4 + 40] ^= 0x33
    p2 = str(tmp_path / "two_bad.dpuf")
    bad2.tofile(p2)
    with pytest.raises(RuntimeError):
        M.Model.open(p2, verify=True)
    # without verification the file still opens (the reference CLI's default)
    M.Model.open(p2, verify=False).close()


def test_container_header_checks(tmp_path):
    m = M.Model.build(TINY, max_seq_len=32, seed=22)
    path = str(tmp_path / "t.dpuf")
    m.save(path)
    raw = np.fromfile(path, np.uint8)
    assert raw[:8].tobytes() == b"DPUF0001"
    hlen = int(raw[20:24].view(np.uint32)[0])
    assert (24 + hlen) % 64 == 0  # payload 64-byte aligned
    bad = raw.copy()
    bad[30] ^= 1  # inside the JSON header -> header CRC mismatch
    p = str(tmp_path / "bad_hdr.dpuf")
    bad.tofile(p)
    with pytest.raises(RuntimeError, match="status -4"):
        M.Model.open(p)
