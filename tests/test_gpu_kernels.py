"""GPU parity of the mode 12 kernels behind the standalone C ABI entry points
against the CPU oracle: bit-exact for the integer/packed work, and for the
fp32 chains whose order the reference fixes."""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import model as M

pytestmark = pytest.mark.gpu

SHAPES = [(16, 64), (40, 128), (200, 1024), (1000, 3072)]
# Qwen3-8B GEMV shapes (rows, cols): K/V, down, gate/up, Q/O
SHAPES_8B = [(1024, 4096), (4096, 12288), (12288, 4096), (4096, 4096)]


def _mat(rows, cols, seed, std=0.02):
    W = M.random_normal(rows * cols, std, seed, f"w{rows}x{cols}").reshape(rows, cols)
    sb = M.sign_bits(cols, seed, f"s{rows}x{cols}")
    blob, d = M.pack_matrix(W, sb)
    return blob, d


def _x(rows, cols, seed):
    return np.random.default_rng(seed).standard_normal((rows, cols)).astype(np.float32)


def _same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.mark.parametrize("rows,cols", SHAPES + SHAPES_8B)
@pytest.mark.parametrize("m", [1, 7])
def test_matmul_f32_bit_exact(eng, orc, rows, cols, m):
    """M = 1 through the one-row GEMV; M = 7 through the few-token GEMMs
    (at the 8B shapes: fragment pairs for 12288 rows, the K-split kernels for
    the others)."""
    blob, d = _mat(rows, cols, 11 + rows)
    x = _x(m, cols, rows + cols)
    # a block with amax <= 1e-4 exercises the zero-scale path
    x[0, :32] = 1e-6
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"matmul_f32 rows={rows} cols={cols} M={m}", flush=True)
    eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                            d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert np.isfinite(out_o).all()
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


def test_matmul_down_8b_dead_zone(eng, orc):
    """The down projection's shape [12288 -> 4096] at M = 1 with its input
    through the SwiGLU dead zone (|x| < 0.005 -> 0, dpuf_engine.c:983-987),
    x shaped like SwiGLU outputs (products of two N(0, 1) halves, scaled):
    zero and near-zero blocks as the real input has them."""
    rows, cols = 4096, 12288
    blob, d = _mat(rows, cols, 61)
    rng = np.random.default_rng(62)
    x = (rng.standard_normal((1, cols)) * rng.standard_normal((1, cols)) * 0.02).astype(np.float32)
    x[np.abs(x) < 0.005] = 0.0
    x[0, 64:96] = 0.0  # a whole zero block
    print(f"down + dead zone: {np.mean(x == 0):.2f} of the input is zero", flush=True)
    out_g = np.full((1, rows), np.nan, np.float32)
    out_o = np.full((1, rows), np.nan, np.float32)
    eng.dpuf_matmul_qr_hadamard4_packed_f32(1, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                            d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_f32(1, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.timeout(600)
@pytest.mark.parametrize("rows,cols", [(12288, 4096), (4096, 12288)])
def test_gemm_m512_8b_shapes(eng, orc, rows, cols):
    """M = 512, the prefill GEMM at the Qwen3-8B gate/up and down shapes;
    the down shape also pruned to its first 224 of 256 tiles through the
    tile-range entry (slab-layout inputs), the prefill's 56/64 pruning."""
    blob, d = _mat(rows, cols, 71 + rows)
    m = 512
    x = _x(m, cols, 72 + rows)
    x[3, 32:64] = 1e-6
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"matmul_f32 rows={rows} cols={cols} M=512", flush=True)
    eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                            d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"
    if rows != 4096:
        return
    nb = cols // 32
    ns = (m + 5) // 6
    sq = np.zeros(ns * nb * 192, np.int8)
    ss = np.zeros(ns * nb * 6, np.float32)
    sm = np.zeros(ns * nb * 6, np.int32)
    for sl in range(ns):
        mc = min(6, m - 6 * sl)
        orc.orc_prep_slab(mc, cols, M.ptr(np.ascontiguousarray(x[6 * sl:6 * sl + mc])), d.sign_bits,
                          M.ptr(sq[sl * nb * 192:]), M.ptr(ss[sl * nb * 6:]), M.ptr(sm[sl * nb * 6:]))
    print("tile range [0, 224) of the down shape, M=512", flush=True)
    out_t = np.full((m, rows), 7.0, np.float32)
    eng.dpuf_matmul_qr_hadamard4_packed_tile_range(m, rows, cols, 0, 224, M.ptr(sq), M.ptr(ss), M.ptr(sm),
                                                   d.tensor_base, d.tile_offsets, M.ptr(out_t))
    assert _same_bits(out_t[:, :224 * 16], out_o[:, :224 * 16])
    assert (out_t[:, 224 * 16:] == 7.0).all()


@pytest.mark.parametrize("cols", [320, 1088, 3072])
@pytest.mark.parametrize("cap", [1, 3, 7])
def test_matmul_skinny_workgroup_caps(eng, orc, cols, cap):
    """The persistent K-split GEMM (2 <= M <= 16, K <= 4096) with its
    workgroups capped so each walks many 16-row fragments through one
    register ring, at 1, 2 and 3 rounds of 32 blocks per fragment."""
    rows, m = 1000, 6
    blob, d = _mat(rows, cols, 81 + cols)
    x = _x(m, cols, 83 + cols)
    x[2, 32:64] = 1e-6
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"skinny rows={rows} cols={cols} M={m} max_workgroups={cap}", flush=True)
    eng.dpuf_amd_set_gemv_max_workgroups(cap)
    try:
        eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                                d.sign_bits, M.ptr(out_g))
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.parametrize("cap", [1, 5])
def test_matmul_few_token_workgroup_caps(eng, orc, cap):
    """The few-token MFMA GEMM (12296 rows: 769 fragments in 385 pairs, the
    last a single group, 2 waves per pair) with its workgroups capped so each
    walks many pairs, restaging nothing between them."""
    rows, cols, m = 12296, 1024, 6
    blob, d = _mat(rows, cols, 91)
    x = _x(m, cols, 93)
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"few-token rows={rows} cols={cols} M={m} max_workgroups={cap}", flush=True)
    eng.dpuf_amd_set_gemv_max_workgroups(cap)
    try:
        eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                                d.sign_bits, M.ptr(out_g))
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.parametrize("rows,cols,m", [(200, 320, 65), (200, 320, 130), (1000, 1024, 130), (72, 64, 200),
                                         (16400, 320, 130), (16384, 4096, 40)])
def test_matmul_token_tiles_bit_exact(eng, orc, rows, cols, m):
    """M > 16: several 64-token tiles of the slab GEMM (the last one ragged),
    partial 64-row tiles, and 10-block rows (a partial last LDS stage); at
    16384 rows and more and M > 128 the 8-wave workgroups (128 rows, the last
    tile partial at 16400 rows)."""
    blob, d = _mat(rows, cols, 31 + rows)
    x = _x(m, cols, 3 * rows + cols)
    x[m - 1, 32:64] = 1e-6  # a zero-scale block in the last tile
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"matmul_f32 rows={rows} cols={cols} M={m}", flush=True)
    eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                            d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert np.isfinite(out_o).all()
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.parametrize("rows,cols,m", [(72, 320, 2), (136, 64, 16), (200, 1088, 16), (1000, 3072, 9),
                                         (4096, 12288, 8), (12288, 4096, 16), (72, 4160, 5),
                                         (200, 320, 17), (1000, 4096, 8), (136, 256, 2), (200, 1024, 5),
                                         (24, 128, 3), (6152, 4096, 7), (24576, 4096, 8), (40000, 256, 3),
                                         (40000, 256, 16), (6152, 4096, 12)])
def test_matmul_skinny_bit_exact(eng, orc, rows, cols, m):
    """M <= 16: the few-token MFMA GEMM (K a multiple of 128 up to 4096 and
    more 16-row fragments than CUs): up to 8 tokens in pairs of fragments
    (24576 and 40000 rows 1 wave per pair, 6152 rows 4 and a last pair with
    one group), 9..16 tokens one fragment per unit (40000 rows 1 wave, 12288
    rows 2, 6152 rows 4); and the K-split GEMMs
    (the rest): odd group counts, a single 4-block quad, block counts that
    are not a multiple of the 32-block round (10, 34, 130: K > 4096 with a
    partial last round), the 8B shapes; M = 17 is the slab GEMM next to it."""
    blob, d = _mat(rows, cols, 41 + rows)
    x = _x(m, cols, 5 * rows + cols)
    x[m - 1, 32:64] = 1e-6  # a zero-scale block
    out_g = np.full((m, rows), np.nan, np.float32)
    out_o = np.full((m, rows), np.nan, np.float32)
    print(f"matmul_f32 rows={rows} cols={cols} M={m}", flush=True)
    eng.dpuf_matmul_qr_hadamard4_packed_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                            d.sign_bits, M.ptr(out_g))
    orc.orc_matmul_f32(m, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert np.isfinite(out_o).all()
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.parametrize("rows,cols", [(24, 192), (8, 320), (1000, 3072), (1024, 4096), (4096, 12288),
                                       (64, 16384)])
@pytest.mark.parametrize("cap", [1, 2, 3, 5, 7, 0])
def test_matmul_m1_workgroup_caps(eng, orc, rows, cols, cap):
    """M = 1 GEMV with the workgroup count capped so each workgroup walks
    several 8-row groups (pipelined loads, chain waves, rotating pair
    buffers); cap 0 is the default launch.  Covers partial 8-block steps
    (cols 192, 320) and the per-round activation path (cols 16384)."""
    blob, d = _mat(rows, cols, 29 + cols)
    x = _x(1, cols, rows * 3 + cols)
    x[0, 32:64] = 1e-6  # a zero-scale block
    out_g = np.full((1, rows), np.nan, np.float32)
    out_o = np.full((1, rows), np.nan, np.float32)
    print(f"matmul M=1 rows={rows} cols={cols} max_workgroups={cap}", flush=True)
    eng.dpuf_amd_set_gemv_max_workgroups(cap)
    try:
        eng.dpuf_matmul_qr_hadamard4_packed_f32(1, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets,
                                                d.sign_bits, M.ptr(out_g))
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)
    orc.orc_matmul_f32(1, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits,
                       M.ptr(out_o))
    assert _same_bits(out_g, out_o), f"max abs diff {np.nanmax(np.abs(out_g - out_o))}"


@pytest.mark.parametrize("cols", [64, 1024, 4096])
def test_fwht_and_prep_row(eng, orc, cols):
    x = _x(1, cols, cols)[0]
    x[:32] *= 1e-7  # zero block
    x[40] = 1e4      # saturating block
    sb = M.sign_bits(cols, 5, "p")
    fg = np.zeros(cols, np.float32)
    fo = np.zeros(cols, np.float32)
    eng.dpuf_fwht64_sign_f32(cols, M.ptr(x), M.ptr(sb), M.ptr(fg))
    orc.orc_fwht64_sign(cols, M.ptr(x), M.ptr(sb), M.ptr(fo))
    assert _same_bits(fg, fo)
    nb = cols // 32
    qg, qo = np.zeros(cols, np.int8), np.zeros(cols, np.int8)
    sg, so = np.zeros(nb, np.float32), np.zeros(nb, np.float32)
    mg, mo = np.zeros(nb, np.int32), np.zeros(nb, np.int32)
    scr = np.zeros(cols, np.float32)
    eng.dpuf_prep_had4_packed_slab(1, cols, M.ptr(x), M.ptr(sb), M.ptr(scr), M.ptr(qg), M.ptr(sg), M.ptr(mg), 0)
    orc.orc_prep_row(cols, M.ptr(x), M.ptr(sb), M.ptr(qo), M.ptr(so), M.ptr(mo))
    assert np.array_equal(qg, qo) and np.array_equal(mg, mo) and _same_bits(sg, so)
    assert _same_bits(scr, fo)


@pytest.mark.parametrize("mc", [1, 4, 6])
def test_prep_slab(eng, orc, mc):
    cols = 256
    nb = cols // 32
    x = _x(mc, cols, 77 + mc)
    sb = M.sign_bits(cols, 9, "slab")
    qg = np.full(nb * 192, 0x55, np.int8)
    sg = np.full(nb * 6, -3.0, np.float32)
    mg = np.full(nb * 6, 99, np.int32)
    qo, so, mo = qg.copy(), sg.copy(), mg.copy()
    scr = np.zeros(mc * cols, np.float32)
    eng.dpuf_prep_had4_packed_slab(mc, cols, M.ptr(x), M.ptr(sb), M.ptr(scr), M.ptr(qg), M.ptr(sg), M.ptr(mg), 1)
    orc.orc_prep_slab(mc, cols, M.ptr(x), M.ptr(sb), M.ptr(qo), M.ptr(so), M.ptr(mo))
    assert np.array_equal(qg, qo) and np.array_equal(mg, mo) and _same_bits(sg, so)


@pytest.mark.parametrize("m", [1, 9])
def test_tile_range(eng, orc, m):
    rows, cols = 100, 512
    blob, d = _mat(rows, cols, 21)
    x = _x(m, cols, 5)
    nb = cols // 32
    # row-layout prep from the oracle, and the slab layout the reference takes for M > 1
    q = np.zeros((m, cols), np.int8)
    s = np.zeros((m, nb), np.float32)
    mm = np.zeros((m, nb), np.int32)
    for i in range(m):
        orc.orc_prep_row(cols, M.ptr(x[i]), d.sign_bits, M.ptr(q[i]), M.ptr(s[i]), M.ptr(mm[i]))
    t0, t1 = 2, 6
    out_g = np.full((m, rows), 7.0, np.float32)
    out_o = np.full((m, rows), 7.0, np.float32)
    orc.orc_gemm_tiles(m, rows, cols, t0, t1, M.ptr(q), M.ptr(s), M.ptr(mm), d.tensor_base, d.tile_offsets,
                       M.ptr(out_o), int(m == 1))
    if m == 1:
        eng.dpuf_matmul_qr_hadamard4_packed_tile_range(1, rows, cols, t0, t1, M.ptr(q), M.ptr(s), M.ptr(mm),
                                                       d.tensor_base, d.tile_offsets, M.ptr(out_g))
    else:
        ns = (m + 5) // 6
        sq = np.zeros(ns * nb * 192, np.int8)
        ss = np.zeros(ns * nb * 6, np.float32)
        sm = np.zeros(ns * nb * 6, np.int32)
        for sl in range(ns):
            mc = min(6, m - 6 * sl)
            orc.orc_prep_slab(mc, cols, M.ptr(np.ascontiguousarray(x[6 * sl:6 * sl + mc])), d.sign_bits,
                              M.ptr(sq[sl * nb * 192:]), M.ptr(ss[sl * nb * 6:]), M.ptr(sm[sl * nb * 6:]))
        eng.dpuf_matmul_qr_hadamard4_packed_tile_range(m, rows, cols, t0, t1, M.ptr(sq), M.ptr(ss), M.ptr(sm),
                                                       d.tensor_base, d.tile_offsets, M.ptr(out_g))
    assert _same_bits(out_g, out_o)
    assert (out_g[:, :t0 * 16] == 7.0).all() and (out_g[:, t1 * 16:] == 7.0).all()


def test_embed(eng, orc):
    rows, cols = 300, 1024
    blob, d = _mat(rows, cols, 31)
    ids = np.array([0, 7, 8, 15, 16, 299, 123], np.int32)
    eg = np.zeros((len(ids), cols), np.float32)
    eo = np.zeros((len(ids), cols), np.float32)
    eng.dpuf_embed_qr_hadamard4_packed_f32(len(ids), cols, M.ptr(ids), d.tensor_base, d.tile_offsets, d.sign_bits,
                                           M.ptr(eg))
    orc.orc_embed(len(ids), cols, M.ptr(ids), d.tensor_base, d.tile_offsets, d.sign_bits, M.ptr(eo))
    assert _same_bits(eg, eo)
    e2 = np.zeros_like(eg)
    eng.dpuf_embed_qr_any_f32(C.byref(d), len(ids), M.ptr(ids), M.ptr(e2), None)
    assert _same_bits(e2, eo)


@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_logit_reductions(eng, orc, offset):
    """Device argmax (first maximum) and Zone-A top-2 exit flag against the
    oracle: rows of every length class (n % 4, shorter than a float4, longer
    than the 64 workgroup slices), 16-byte misaligned starts, ties, a NaN
    first element, repeated maxima."""
    rng = np.random.default_rng(40 + offset)
    cases = []
    for n in (1, 2, 3, 5, 63, 257, 4096, 40961, 151936):
        cases.append(rng.standard_normal(n).astype(np.float32))
        cases.append(rng.integers(-2, 3, n).astype(np.float32))  # many ties
    x = rng.standard_normal(5000).astype(np.float32)
    x[[17, 4000]] = 9.0  # repeated maximum
    cases.append(x)
    x = rng.standard_normal(3000).astype(np.float32)
    x[0] = np.nan
    cases.append(x)
    x = rng.standard_normal(3000).astype(np.float32)
    x[[5, 2999]] = np.nan
    cases.append(x)
    for x in cases:
        n = x.size
        got = eng.dpuf_amd_reduce_check(M.ptr(x), n, offset, 1, 0.0)
        assert got == orc.orc_argmax(M.ptr(x), n), (n, offset)
        for thr in (1e-7, 0.05, 0.5, 3.0):
            got = eng.dpuf_amd_reduce_check(M.ptr(x), n, offset, 0, thr)
            assert got == orc.orc_top2_exit(M.ptr(x), n, thr), (n, offset, thr)


@pytest.mark.parametrize("rows,cols", [(40, 128), (1000, 3072)])
def test_verify_tiles_device(eng, rows, cols):
    """The GPU tile CRC32 check against the host one (reference
    dpuf_avx2.c:846-908): all tiles good, then one corrupted body byte at a
    time (first, a middle and the last tile) flagged by both."""
    blob, d = _mat(rows, cols, 41 + rows)
    n = d.n_tiles
    offs = np.ctypeslib.as_array(C.cast(d.tile_offsets, C.POINTER(C.c_uint64)), (n,)).copy()
    region = blob[C.cast(d.tensor_base, C.c_void_p).value - blob.ctypes.data:].copy()
    ok_h, ok_d = np.zeros(n, np.uint8), np.full(n, 7, np.uint8)
    print(f"verify_tiles rows={rows} cols={cols} tiles={n}", flush=True)
    assert eng.dpuf_qr_verify_tiles_ex(12, n, cols, M.ptr(region), M.ptr(offs), M.ptr(ok_h)) == 0
    assert eng.dpuf_amd_verify_tiles_device(12, n, cols, M.ptr(region), M.ptr(offs), M.ptr(ok_d)) == 0
    assert ok_h.all() and ok_d.all()
    for t, at in ((0, 1), (n // 2, 777 % (cols // 2)), (n - 1, 5)):
        bad = region.copy()
        bad[int(offs[t]) + 16 + at] ^= 0x5A  # 16-byte tile header, then the body
        nh = eng.dpuf_qr_verify_tiles_ex(12, n, cols, M.ptr(bad), M.ptr(offs), M.ptr(ok_h))
        nd = eng.dpuf_amd_verify_tiles_device(12, n, cols, M.ptr(bad), M.ptr(offs), M.ptr(ok_d))
        assert nh == 1 and nd == 1 and ok_d[t] == 0 and np.array_equal(ok_h, ok_d), (t, nh, nd)
