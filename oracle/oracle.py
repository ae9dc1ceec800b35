"""ctypes wrapper of liboracle.so -- the CPU restatement of the reference
Mode 12 token loop.  TEST INFRASTRUCTURE ONLY: imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg as the checker.
"""
import ctypes as C
import os
import subprocess

from dpuf_amd.abi import DpufLayerWeights, DpufModelConfig, DpufWeightDesc

_HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None
P = C.c_void_p
I32 = C.c_int32


def build():
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _sig(lib, name, res, args):
    f = getattr(lib, name)
    f.restype = res
    f.argtypes = args


def load():
    global _lib
    if _lib is not None:
        return _lib
    path = os.path.join(_HERE, "liboracle.so")
    if not os.path.exists(path):
        build()
    lib = C.CDLL(path)
    _sig(lib, "orc_h2f", C.c_float, [C.c_uint16])
    _sig(lib, "orc_exp_poly", C.c_float, [C.c_float])
    _sig(lib, "orc_fwht64", None, [P])
    _sig(lib, "orc_fwht64_sign", None, [I32, P, P, P])
    _sig(lib, "orc_prep_row", None, [I32, P, P, P, P, P])
    _sig(lib, "orc_prep_slab", None, [I32, I32, P, P, P, P, P])
    _sig(lib, "orc_gemm_tiles", None, [I32, I32, I32, I32, I32, P, P, P, P, P, P, C.c_int])
    _sig(lib, "orc_matmul_f32", None, [I32, I32, I32, I32, P, P, P, P, P])
    _sig(lib, "orc_embed", None, [I32, I32, P, P, P, P, P])
    _sig(lib, "orc_gemm_tiles_asym", None, [I32, I32, I32, I32, I32, I32, P, P, P, P, P, P])
    _sig(lib, "orc_matmul_asym_f32", None, [I32, I32, I32, I32, I32, P, P, P, P, P])
    _sig(lib, "orc_embed_asym", None, [I32, I32, I32, P, P, P, P, P])
    _sig(lib, "orc_embed_desc", None, [C.POINTER(DpufWeightDesc), I32, P, P])
    _sig(lib, "orc_add_rmsnorm", None, [I32, P, P, P, C.c_float, P])
    _sig(lib, "orc_rope_tables", None, [C.POINTER(DpufModelConfig), P, P])
    _sig(lib, "orc_rope_apply", None, [I32, P, P, P])
    _sig(lib, "orc_attn_heads", None, [I32, I32, C.c_float, P, P, P, P, P, P, P, P])
    _sig(lib, "orc_swiglu1", C.c_float, [C.c_float, C.c_float, C.c_float])
    _sig(lib, "orc_quant_q8", None, [I32, P, P, P])
    _sig(lib, "orc_attn_heads_q8", None, [I32, I32, C.c_float, P, P, P, P, P, P, P, P, P, P])
    _sig(lib, "orc_engine_create", P, [C.POINTER(DpufModelConfig), C.POINTER(DpufLayerWeights),
                                        C.POINTER(DpufWeightDesc), C.POINTER(DpufWeightDesc), P])
    _sig(lib, "orc_engine_destroy", None, [P])
    _sig(lib, "orc_engine_set_slot", I32, [P, I32])
    _sig(lib, "orc_engine_reset_slot", None, [P, I32])
    _sig(lib, "orc_engine_freeze_prefix", I32, [P, I32, I32])
    _sig(lib, "orc_engine_apply_prefix", I32, [P, I32, I32])
    _sig(lib, "orc_engine_set_kv", I32, [P, I32, I32, I32, I32, P, P])
    _sig(lib, "orc_engine_get_kv", I32, [P, I32, I32, I32, I32, P, P])
    _sig(lib, "orc_engine_set_capture", None, [P, I32])
    _sig(lib, "orc_engine_get_capture", P, [P])
    _sig(lib, "orc_engine_forward", I32, [P, I32, P, I32, P, I32, P])
    _sig(lib, "orc_argmax", I32, [P, I32])
    _sig(lib, "orc_top2_exit", I32, [P, I32, C.c_float])
    _sig(lib, "orc_num_threads", I32, [])
    _sig(lib, "orc_set_num_threads", None, [I32])
    _sig(lib, "orc_set_norm_order", None, [I32])
    _lib = lib
    return lib
