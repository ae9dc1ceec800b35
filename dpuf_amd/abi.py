"""ctypes mirror of the DPUF C ABI (include/dpuf_kernels.h) and loaders.

The structures below have the byte layout of the reference header
(dpuf_kernels.h:44-101 in dulePan/dpuf; the reference's own ctypes mirror is
dpuf_format.py:2060-2127): DpufWeightDesc 48 bytes, DpufModelConfig 92 bytes,
DpufLayerWeights 368 bytes.
"""
import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))


class DpufWeightDesc(C.Structure):
    _fields_ = [
        ("mode", C.c_int32),
        ("rows", C.c_int32),
        ("cols", C.c_int32),
        ("n_tiles", C.c_int32),
        ("tensor_base", C.c_void_p),
        ("tile_offsets", C.c_void_p),
        ("col_scale", C.c_void_p),
        ("sign_bits", C.c_void_p),
    ]


class DpufModelConfig(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32),
        ("num_layers", C.c_int32),
        ("num_q_heads", C.c_int32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("vocab_size", C.c_int32),
        ("max_seq_len", C.c_int32),
        ("has_qk_norm", C.c_int32),
        ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("n_threads", C.c_int32),
        ("use_llama3_rope", C.c_int32),
        ("rope_factor", C.c_float),
        ("rope_low_freq", C.c_float),
        ("rope_high_freq", C.c_float),
        ("rope_orig_max_pos", C.c_int32),
        ("kv_type", C.c_int32),
        ("has_mrope", C.c_int32),
        ("mrope_section", C.c_int32 * 3),
        ("mrope_interleaved", C.c_int32),
    ]


class DpufLayerWeights(C.Structure):
    _fields_ = [
        ("attn_norm", C.c_void_p),
        ("attn_q_norm", C.c_void_p),
        ("attn_k_norm", C.c_void_p),
        ("ffn_norm", C.c_void_p),
        ("w_q", DpufWeightDesc),
        ("w_k", DpufWeightDesc),
        ("w_v", DpufWeightDesc),
        ("w_o", DpufWeightDesc),
        ("w_gate", DpufWeightDesc),
        ("w_up", DpufWeightDesc),
        ("w_down", DpufWeightDesc),
    ]


assert C.sizeof(DpufWeightDesc) == 48
assert C.sizeof(DpufModelConfig) == 92
assert C.sizeof(DpufLayerWeights) == 368


class DpufToolsSpec(C.Structure):
    _fields_ = [
        ("hidden_size", C.c_int32),
        ("intermediate_size", C.c_int32),
        ("num_layers", C.c_int32),
        ("num_q_heads", C.c_int32),
        ("num_kv_heads", C.c_int32),
        ("head_dim", C.c_int32),
        ("vocab_size", C.c_int32),
        ("max_seq_len", C.c_int32),
        ("tie_word_embeddings", C.c_int32),
        ("weight_std", C.c_float),
        ("rms_eps", C.c_float),
        ("rope_theta", C.c_float),
        ("seed", C.c_uint64),
        ("weight_plan", C.c_int32),
    ]


P = C.c_void_p
I32 = C.c_int32
F32P = C.POINTER(C.c_float)


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args
    return f


def lib_path(name):
    return os.path.join(_HERE, name)


_tools = None
_engine = None


def load_tools():
    """libdpuf_tools.so: packer, container writer/reader (host C only)."""
    global _tools
    if _tools is not None:
        return _tools
    path = lib_path("libdpuf_tools.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(path)
    _sig(lib, "dpuf_tools_random_normal", None, [P, C.c_size_t, C.c_float, C.c_uint64, C.c_char_p])
    _sig(lib, "dpuf_tools_round_bf16", None, [P, C.c_size_t])
    _sig(lib, "dpuf_tools_f32_to_f16", C.c_uint16, [C.c_float])
    _sig(lib, "dpuf_tools_f16_to_f32", C.c_float, [C.c_uint16])
    _sig(lib, "dpuf_tools_sign_bits", None, [P, I32, C.c_uint64, C.c_char_p])
    _sig(lib, "dpuf_tools_pack_mode12", P, [P, I32, I32, P, I32, C.POINTER(C.c_size_t)])
    _sig(lib, "dpuf_tools_pack_asym", P, [P, I32, I32, P, I32, I32, C.c_float, C.POINTER(C.c_size_t)])
    _sig(lib, "dpuf_tools_bind_blob", I32, [P, C.c_size_t, C.POINTER(DpufWeightDesc)])
    _sig(lib, "dpuf_tools_pack_raw_tiny", P, [P, I32, C.POINTER(C.c_size_t)])
    _sig(lib, "dpuf_tools_build_model", P, [C.POINTER(DpufToolsSpec)])
    _sig(lib, "dpuf_tools_save_container", C.c_uint64, [P, C.c_char_p])
    _sig(lib, "dpuf_tools_open_container", P, [C.c_char_p, I32, I32, C.POINTER(I32)])
    _sig(lib, "dpuf_tools_free_model", None, [P])
    _sig(lib, "dpuf_tools_model_cfg", C.POINTER(DpufModelConfig), [P])
    _sig(lib, "dpuf_tools_model_layers", C.POINTER(DpufLayerWeights), [P])
    _sig(lib, "dpuf_tools_model_tok", C.POINTER(DpufWeightDesc), [P])
    _sig(lib, "dpuf_tools_model_lm", C.POINTER(DpufWeightDesc), [P])
    _sig(lib, "dpuf_tools_model_out_norm", P, [P])
    _sig(lib, "dpuf_tools_model_healed", I32, [P])
    _sig(lib, "dpuf_tools_model_weight_bytes", C.c_uint64, [P])
    _sig(lib, "dpuf_crc32_bytes", C.c_uint32, [P, C.c_uint32])
    _sig(lib, "dpuf_qr_verify_tiles_ex", I32, [I32, I32, I32, P, P, P])
    libc = C.CDLL(None)
    lib._free = _sig(libc, "free", None, [P])
    _tools = lib
    return lib


ENGINE_SYMBOLS = [
    "dpuf_crc32_bytes", "dpuf_qr_verify_tiles", "dpuf_qr_verify_tiles_ex",
    "dpuf_fwht64_sign_f32", "dpuf_prep_had4_packed_slab",
    "dpuf_matmul_qr_hadamard4_packed_tile_range", "dpuf_matmul_qr_hadamard4_packed_f32",
    "dpuf_embed_qr_hadamard4_packed_f32", "dpuf_embed_qr_any_f32",
    "dpuf_matmul_qr_had4_asym_tile_range", "dpuf_matmul_qr_had4_asym_f32", "dpuf_embed_qr_had4_asym_f32",
    "dpuf_matmul_qr_had6_tile_range", "dpuf_matmul_qr_had6_f32", "dpuf_embed_qr_had6_f32",
    "dpuf_engine_create", "dpuf_engine_destroy", "dpuf_engine_reset_cache",
    "dpuf_engine_set_slot", "dpuf_engine_get_slot", "dpuf_engine_reset_slot",
    "dpuf_engine_slot_memory", "dpuf_engine_num_slots", "dpuf_engine_freeze_prefix",
    "dpuf_engine_apply_prefix", "dpuf_engine_get_prefix_len",
    "dpuf_engine_forward_batch", "dpuf_engine_forward_batch_ex", "dpuf_engine_forward_token",
]


def load_engine():
    """libdpuf_amd.so: the HIP engine behind the C ABI.  Raises if missing."""
    global _engine
    if _engine is not None:
        return _engine
    path = lib_path("libdpuf_amd.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() first")
    lib = C.CDLL(path)
    _sig(lib, "dpuf_crc32_bytes", C.c_uint32, [P, C.c_uint32])
    _sig(lib, "dpuf_qr_verify_tiles_ex", I32, [I32, I32, I32, P, P, P])
    _sig(lib, "dpuf_fwht64_sign_f32", None, [I32, P, P, P])
    _sig(lib, "dpuf_prep_had4_packed_slab", None, [I32, I32, P, P, P, P, P, P, I32])
    _sig(lib, "dpuf_matmul_qr_hadamard4_packed_tile_range", None,
         [I32, I32, I32, I32, I32, P, P, P, P, P, P])
    _sig(lib, "dpuf_matmul_qr_hadamard4_packed_f32", None, [I32, I32, I32, I32, P, P, P, P, P])
    _sig(lib, "dpuf_embed_qr_hadamard4_packed_f32", None, [I32, I32, P, P, P, P, P])
    _sig(lib, "dpuf_embed_qr_any_f32", None, [C.POINTER(DpufWeightDesc), I32, P, P, P])
    for mode in ("had4_asym", "had6"):
        _sig(lib, f"dpuf_matmul_qr_{mode}_tile_range", None, [I32, I32, I32, I32, I32, P, P, P, P, P, P])
        _sig(lib, f"dpuf_matmul_qr_{mode}_f32", None, [I32, I32, I32, I32, P, P, P, P, P])
        _sig(lib, f"dpuf_embed_qr_{mode}_f32", None, [I32, I32, P, P, P, P, P])
    _sig(lib, "dpuf_engine_create", P, [C.POINTER(DpufModelConfig), C.POINTER(DpufLayerWeights),
                                         C.POINTER(DpufWeightDesc), C.POINTER(DpufWeightDesc), P])
    _sig(lib, "dpuf_engine_destroy", None, [P])
    _sig(lib, "dpuf_engine_reset_cache", None, [P])
    _sig(lib, "dpuf_engine_set_slot", I32, [P, I32])
    _sig(lib, "dpuf_engine_get_slot", I32, [P])
    _sig(lib, "dpuf_engine_reset_slot", None, [P, I32])
    _sig(lib, "dpuf_engine_slot_memory", C.c_size_t, [P])
    _sig(lib, "dpuf_engine_num_slots", I32, [P])
    _sig(lib, "dpuf_engine_freeze_prefix", I32, [P, I32, I32])
    _sig(lib, "dpuf_engine_apply_prefix", I32, [P, I32, I32])
    _sig(lib, "dpuf_engine_get_prefix_len", I32, [P, I32])
    _sig(lib, "dpuf_engine_forward_batch", I32, [P, I32, P, I32, I32, P])
    _sig(lib, "dpuf_engine_forward_batch_ex", I32, [P, I32, P, I32, P, P, P, P, P, I32, P])
    _sig(lib, "dpuf_engine_forward_token", I32, [P, I32, I32, P])
    # additive entry points (include/dpuf_amd.h)
    _sig(lib, "dpuf_amd_device_ok", I32, [])
    _sig(lib, "dpuf_amd_last_error", C.c_char_p, [])
    _sig(lib, "dpuf_amd_engine_forward_argmax", I32, [P, I32, P, I32, P, I32, P, P])
    _sig(lib, "dpuf_amd_engine_set_kv", I32, [P, I32, I32, I32, I32, P, P])
    _sig(lib, "dpuf_amd_engine_get_kv", I32, [P, I32, I32, I32, I32, P, P])
    _sig(lib, "dpuf_amd_engine_set_capture", I32, [P, I32])
    _sig(lib, "dpuf_amd_engine_get_capture", I32, [P, P, C.c_size_t])
    _sig(lib, "dpuf_amd_engine_set_timing", None, [P, I32])
    _sig(lib, "dpuf_amd_engine_set_graphs", None, [P, I32])
    _sig(lib, "dpuf_amd_engine_get_timing", I32, [P, I32, C.POINTER(C.c_double), C.POINTER(C.c_int64),
                                                  C.POINTER(C.c_double)])
    _sig(lib, "dpuf_amd_engine_weight_bytes", C.c_uint64, [P])
    _sig(lib, "dpuf_amd_engine_early_exit_count", C.c_int64, [P])
    _sig(lib, "dpuf_amd_attn_path_count", C.c_int64, [I32])
    _sig(lib, "dpuf_amd_gemv_bench", C.c_double, [P, I32, I32, I32, I32, C.POINTER(C.c_double)])
    _sig(lib, "dpuf_amd_copy_bench", C.c_double, [C.c_size_t, I32])
    _sig(lib, "dpuf_amd_set_gemv_max_workgroups", None, [I32])
    _sig(lib, "dpuf_amd_reduce_check", I32, [P, I32, I32, I32, C.c_float])
    _sig(lib, "dpuf_amd_reduce_check_noalloc", I32, [P, I32, I32, C.c_float, P, P])
    _sig(lib, "dpuf_amd_verify_tiles_device", I32, [I32, I32, I32, P, P, P])
    _sig(lib, "dpuf_amd_engine_forward_slots", I32, [P, I32, P, P, P, P, P])
    _engine = lib
    return lib
