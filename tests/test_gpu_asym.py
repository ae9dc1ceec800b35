"""GPU parity of Modes 13 / 14 (asymmetric blk64 4-bit and 6-bit, reference
dpuf_avx2.c:2785-3221) against the CPU oracle, through the C ABI: the
standalone GEMV / GEMM, tile-range and embedding entries at small and
Qwen3-8B shapes, and the engine over models packed with the had4p-hybrid
plan (pack_dpuf.py:249-266).  Bit for bit."""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import model as M
from test_gpu_configs import Pair, bits_equal, greedy, log, maxdiff

pytestmark = pytest.mark.gpu

NAMES = {13: "had4_asym", 14: "had6"}


def _mat(rows, cols, seed, mode):
    W = M.random_normal(rows * cols, 0.02, seed, f"a{rows}x{cols}").reshape(rows, cols)
    sb = M.sign_bits(cols, seed, f"as{rows}x{cols}")
    blob, d = M.pack_matrix(W, sb, mode=mode)
    return blob, d


def _run(eng, orc, d, x):
    m, rows, cols = x.shape[0], d.rows, d.cols
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    getattr(eng, f"dpuf_matmul_qr_{NAMES[d.mode]}_f32")(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base,
                                                        d.tile_offsets, d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_asym_f32(int(d.mode == 14), m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                            d.sign_bits, M.ptr(out_o))
    assert np.isfinite(out_o).all()
    return out_g, out_o


@pytest.mark.parametrize("mode", [13, 14])
@pytest.mark.parametrize("rows,cols,m", [(40, 256, 1), (200, 1024, 1), (1000, 3072, 1), (40, 256, 3),
                                         (200, 1024, 17), (72, 512, 64), (200, 320 + 64, 130)])
def test_matmul_bit_exact(eng, orc, mode, rows, cols, m):
    """M = 1 (the GEMV with its DPP pair exchange) and M > 1 (the MFMA GEMM
    with the 64-block epilogue): partial tiles, ragged token tiles, a zero
    block."""
    blob, d = _mat(rows, cols, 5 + rows + mode, mode)
    x = np.random.default_rng(rows + cols + m).standard_normal((m, cols)).astype(np.float32)
    x[0, :32] = 1e-6
    log(f"mode {mode} rows={rows} cols={cols} M={m}")
    g, o = _run(eng, orc, d, x)
    assert bits_equal(g, o), maxdiff(g, o)


@pytest.mark.parametrize("mode", [13, 14])
@pytest.mark.parametrize("rows,cols", [(1024, 4096), (4096, 12288), (12288, 4096), (4096, 4096)])
def test_matmul_8b_shapes_m1(eng, orc, mode, rows, cols):
    """The Qwen3-8B GEMV shapes (K/V, down, gate/up, Q/O) at M = 1."""
    blob, d = _mat(rows, cols, 17 + rows, mode)
    x = np.random.default_rng(rows * 3 + cols).standard_normal((1, cols)).astype(np.float32)
    log(f"mode {mode} 8B shape rows={rows} cols={cols} M=1")
    g, o = _run(eng, orc, d, x)
    assert bits_equal(g, o), maxdiff(g, o)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("mode", [13, 14])
def test_gemm_m512_and_tile_range(eng, orc, mode):
    """M = 512 at the down shape [12288 -> 4096] and its first 224 tiles
    through the tile-range entry with slab-layout inputs."""
    rows, cols, m = 4096, 12288, 512
    blob, d = _mat(rows, cols, 31 + mode, mode)
    x = np.random.default_rng(32).standard_normal((m, cols)).astype(np.float32)
    log(f"mode {mode} M=512 rows={rows} cols={cols}")
    g, o = _run(eng, orc, d, x)
    assert bits_equal(g, o), maxdiff(g, o)
    nb, ns = cols // 32, (m + 5) // 6
    sq = np.zeros(ns * nb * 192, np.int8)
    ss = np.zeros(ns * nb * 6, np.float32)
    sm = np.zeros(ns * nb * 6, np.int32)
    for sl in range(ns):
        mc = min(6, m - 6 * sl)
        orc.orc_prep_slab(mc, cols, M.ptr(np.ascontiguousarray(x[6 * sl:6 * sl + mc])), d.sign_bits,
                          M.ptr(sq[sl * nb * 192:]), M.ptr(ss[sl * nb * 6:]), M.ptr(sm[sl * nb * 6:]))
    log(f"mode {mode} tile range [0, 224), M=512")
    out_t = np.full((m, rows), 7.0, np.float32)
    getattr(eng, f"dpuf_matmul_qr_{NAMES[mode]}_tile_range")(m, rows, cols, 0, 224, M.ptr(sq), M.ptr(ss), M.ptr(sm),
                                                             d.tensor_base, d.tile_offsets, M.ptr(out_t))
    assert bits_equal(out_t[:, :224 * 16], o[:, :224 * 16])
    assert (out_t[:, 224 * 16:] == 7.0).all()


@pytest.mark.parametrize("mode", [13, 14])
def test_tile_range_m1_and_embed(eng, orc, mode):
    """The M = 1 tile-range entry (row-layout prep) over tiles [2, 9), and
    embedding rows through the mode's own entry and the dispatcher."""
    rows, cols = 200, 1024
    blob, d = _mat(rows, cols, 41 + mode, mode)
    x = np.random.default_rng(42).standard_normal(cols).astype(np.float32)
    nb = cols // 32
    q = np.zeros(cols, np.int8)
    s = np.zeros(nb, np.float32)
    m = np.zeros(nb, np.int32)
    orc.orc_prep_row(cols, M.ptr(x), d.sign_bits, M.ptr(q), M.ptr(s), M.ptr(m))
    out_g = np.full(rows, 5.0, np.float32)
    out_o = np.full(rows, 5.0, np.float32)
    getattr(eng, f"dpuf_matmul_qr_{NAMES[mode]}_tile_range")(1, rows, cols, 2, 9, M.ptr(q), M.ptr(s), M.ptr(m),
                                                             d.tensor_base, d.tile_offsets, M.ptr(out_g))
    orc.orc_gemm_tiles_asym(int(mode == 14), 1, rows, cols, 2, 9, M.ptr(q), M.ptr(s), M.ptr(m), d.tensor_base,
                            d.tile_offsets, M.ptr(out_o))
    assert bits_equal(out_g, out_o)
    assert (out_g[:32] == 5).all() and (out_g[144:] == 5).all()
    ids = np.array([0, 7, 8, 15, 16, 199, 100], np.int32)
    eg = np.zeros((len(ids), cols), np.float32)
    ea = np.zeros((len(ids), cols), np.float32)
    eo = np.zeros((len(ids), cols), np.float32)
    getattr(eng, f"dpuf_embed_qr_{NAMES[mode]}_f32")(len(ids), cols, M.ptr(ids), d.tensor_base, d.tile_offsets,
                                                     d.sign_bits, M.ptr(eg))
    eng.dpuf_embed_qr_any_f32(C.byref(d), len(ids), M.ptr(ids), M.ptr(ea), None)
    orc.orc_embed_asym(int(mode == 14), len(ids), cols, M.ptr(ids), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(eo))
    assert bits_equal(eg, eo) and bits_equal(ea, eo)


HYB = dict(hidden_size=256, intermediate_size=512, num_layers=3, num_q_heads=8, num_kv_heads=2, head_dim=64,
           vocab_size=4096, tie_word_embeddings=0)


@pytest.mark.parametrize("heads", [(4, 2), (8, 2)])
def test_engine_hybrid_prefill_decode(eng, orc, heads, monkeypatch):
    """A model packed with the had4p-hybrid plan (token embedding and most
    matrices mode 13; K, V, down, even-layer O and the LM head mode 14; every
    matrix with its own signs, so Q/K/V take three preps): a 13-token
    prefill with per-layer residuals, 10 greedy steps, then 3 steps through
    the captured-graph device-argmax entry; and the down projection pruned."""
    monkeypatch.setenv("DPUF_GEN_KEEP_TILES", "12")
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "12")
    nq, nkv = heads
    m = M.Model.build(dict(HYB, num_q_heads=nq, num_kv_heads=nkv), max_seq_len=64, seed=301, weight_plan=1)
    assert m.tok.contents.mode == 13 and m.lm.contents.mode == 14
    p = Pair(eng, orc, m)
    p.capture(16)
    ids = np.random.default_rng(302).integers(0, 4096, 13).astype(np.int32)
    log(f"hybrid heads={heads}: prefill 13")
    lg, lo = p.forward(ids, 0, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(13)
    assert bits_equal(cg, co), maxdiff(cg, co)
    toks, _ = greedy(p, lg, lo, 13, 10, "hybrid")
    # positions 13 .. 22 are cached; three more steps through the graph entry
    tok, out = toks[-1], C.c_int32(-1)
    for s in range(3):
        pos = 23 + s
        log(f"hybrid graph step at {pos}")
        ref = np.zeros(4096, np.float32)
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1,
                                                C.byref(out), None)
        assert rc == 0
        assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1, M.ptr(ref)) == 0
        assert out.value == orc.orc_argmax(M.ptr(ref), 4096)
        tok = out.value
    p.close()


@pytest.mark.timeout(600)
def test_engine_hybrid_8b_widths(eng, orc):
    """Hybrid plan at the Qwen3-8B widths (hidden 4096, FFN 12288, 32 / 8
    heads of 128; 2 layers, vocab 32768): the mode 14 down projection at
    K = 12288 and the mode 13 gate/up at 12288 rows in the engine, prefill of
    40 tokens (the MFMA GEMM) and 6 greedy steps (the GEMV)."""
    shape = dict(hidden_size=4096, intermediate_size=12288, num_layers=2, num_q_heads=32, num_kv_heads=8,
                 head_dim=128, vocab_size=32768, tie_word_embeddings=0)
    log("building the hybrid 8B-width model")
    m = M.Model.build(shape, max_seq_len=64, seed=311, weight_plan=1)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(312).integers(0, 32768, 40).astype(np.int32)
    log("hybrid 8B widths: prefill 40")
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 40, 6, "hybrid 8B")
    p.close()
