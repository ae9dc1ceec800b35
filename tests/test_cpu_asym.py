"""Pins the oracle's Modes 13 / 14 (asymmetric blk64 4-bit and 6-bit,
reference dpuf_avx2.c:2785-3221) and this repository's packer for them.

Tiles are built here by an independent constructor that follows the
reference packer's array steps (dpuf_format.py:1688-1725: the dm block, the
q4 nibble interleave, the q2 2-bit planes) from chosen codes q, d, m.  The
oracle's embedding and GEMV of those tiles must then equal closed forms in
float64:

    row r (rotated)  = m[r, g] + q[r, j] * d[r, g]        (then FWHT-64, signs)
    y[r]             = sum_g d[r, g] (D0 xs0 + D1 xs1) + m[r, g] (S0 xs0 + S1 xs1)

with D the integer dots of the two 32-blocks of g, S the sums of the int8
activations of each block and xs their scales.  A mistake the restatement
could make -- d and m swapped, the 2-bit planes dropped or read for the wrong
row, nibble halves swapped, the activation sum taken without its 1/8 -- is
planted in the closed form or the constructor and must move the result far
outside the bound.  CPU only.
"""
import ctypes as C
import struct

import numpy as np
import pytest

from dpuf_amd import model as M


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def build_tiles(q, d16, m16, bits, row_plane_swap=False):
    """Tile region and offsets for codes q [rows, cols] (0 .. 2^bits - 1) and
    fp16 d, m [rows, cols / 64].  row_plane_swap builds the 2-bit planes with
    the two row-index halves exchanged (a layout mistake to catch)."""
    rows, cols = q.shape
    n_64, n_blk = cols // 64, cols // 32
    out, offs = bytearray(), [0]
    for t0 in range(0, rows, 16):
        n_r = min(16, rows - t0)
        n_8g = (n_r + 7) // 8
        qp = np.zeros((n_8g * 8, cols), np.uint8)
        dp = np.zeros((n_8g * 8, n_64), np.float16)
        mp = np.zeros((n_8g * 8, n_64), np.float16)
        qp[:n_r], dp[:n_r], mp[:n_r] = q[t0:t0 + n_r], d16[t0:t0 + n_r], m16[t0:t0 + n_r]
        dm = np.empty((n_8g, n_64, 16), np.float16)
        dm[:, :, :8] = dp.reshape(n_8g, 8, n_64).transpose(0, 2, 1)
        dm[:, :, 8:] = mp.reshape(n_8g, 8, n_64).transpose(0, 2, 1)
        # (group, row, block, chunk, half, k) -> bytes (group, block, chunk, row, k)
        lo = (qp & 15).reshape(n_8g, 8, n_blk, 4, 2, 4)
        q4 = ((lo[..., 1, :] << 4) | lo[..., 0, :]).transpose(0, 2, 3, 1, 4)
        if bits == 6:
            # row = 2a + b: (group, a, b, block, chunk, half, k) -> (group, a, block, chunk, half, b, k)
            hi = ((qp >> 4) & 3).reshape(n_8g, 4, 2, n_blk, 4, 2, 4)
            if row_plane_swap:
                hi = ((qp >> 4) & 3).reshape(n_8g, 2, 4, n_blk, 4, 2, 4).transpose(0, 2, 1, 3, 4, 5, 6)
            ht = hi.transpose(0, 1, 3, 4, 5, 2, 6)
            q2 = ht[:, 0] | (ht[:, 1] << 2) | (ht[:, 2] << 4) | (ht[:, 3] << 6)
        body = b"".join(dm[g].tobytes() + q4[g].astype(np.uint8).tobytes() +
                        (q2[g].astype(np.uint8).tobytes() if bits == 6 else b"") for g in range(n_8g))
        tile = struct.pack("<IHHII", 0, n_r, 0, 0, 0) + body
        tile += b"\0" * ((64 - len(tile) % 64) % 64)
        out += tile
        offs.append(len(out))
    return np.frombuffer(bytes(out), np.uint8).copy(), np.array(offs, np.uint64)


def random_codes(rows, cols, bits, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 1 << bits, (rows, cols)).astype(np.uint8)
    d16 = rng.uniform(0.001, 0.01, (rows, cols // 64)).astype(np.float16)
    m16 = rng.uniform(-0.05, 0.05, (rows, cols // 64)).astype(np.float16)
    return q, d16, m16


def signs_of(sb, cols):
    return np.where(np.unpackbits(sb, bitorder="little")[:cols].astype(bool), -1.0, 1.0)


def hadamard64():
    H = np.array([[1.0]])
    while H.shape[0] < 64:
        H = np.block([[H, H], [H, -H]])
    return H / 8.0


def embed_closed(q, d16, m16, sb):
    rows, cols = q.shape
    v = (q.astype(np.float32) * np.repeat(d16.astype(np.float32), 64, axis=1)).astype(np.float32)
    v = (v + np.repeat(m16.astype(np.float32), 64, axis=1)).astype(np.float32)
    Hm = hadamard64()
    out = (v.astype(np.float64).reshape(rows, -1, 64) @ Hm.T).reshape(rows, cols)
    return out * signs_of(sb, cols)


def oracle_embed(orc, tiles, offs, sb, bits, cols, ids):
    ids = np.ascontiguousarray(ids, np.int32)
    out = np.zeros((len(ids), cols), np.float32)
    orc.orc_embed_asym(int(bits == 6), len(ids), cols, M.ptr(ids), M.ptr(tiles), M.ptr(offs), M.ptr(sb), M.ptr(out))
    return out


def oracle_prep(orc, x, sb):
    Mt, K = x.shape
    q = np.zeros((Mt, K), np.int8)
    s = np.zeros((Mt, K // 32), np.float32)
    m = np.zeros((Mt, K // 32), np.int32)
    for i in range(Mt):
        orc.orc_prep_row(K, M.ptr(f32(x[i])), M.ptr(sb), M.ptr(q[i]), M.ptr(s[i]), M.ptr(m[i]))
    return q, s, m


def oracle_gemv(orc, tiles, offs, bits, rows, cols, q, s, m, t0=0, t1=None, fill=0.0):
    t1 = (rows + 15) // 16 if t1 is None else t1
    out = np.full((q.shape[0], rows), fill, np.float32)
    orc.orc_gemm_tiles_asym(int(bits == 6), q.shape[0], rows, cols, t0, t1, M.ptr(q), M.ptr(s), M.ptr(m),
                            M.ptr(tiles), M.ptr(offs), M.ptr(out))
    return out


def gemv_closed(qw, d16, m16, xq, xs, mut=()):
    """float64 y[token, row] from the codes; `mut` plants one mistake."""
    rows, cols = qw.shape
    qwf = qw.astype(np.float64)
    if "halves_swapped" in mut:  # columns 8c+k <-> 8c+4+k
        qwf = qwf.reshape(rows, -1, 2, 4)[:, :, ::-1, :].reshape(rows, cols)
    if "no_high_bits" in mut:
        qwf = (qw & 15).astype(np.float64)
    d = d16.astype(np.float64)
    m = m16.astype(np.float64)
    if "d_m_swapped" in mut:
        d, m = m, d
    y = np.zeros((xq.shape[0], rows))
    for t in range(xq.shape[0]):
        xb = xq[t].astype(np.float64).reshape(-1, 32)
        D = (qwf.reshape(rows, -1, 32) * xb[None]).sum(axis=2)          # [rows, n_blk]
        S = xb.sum(axis=1) * (8.0 if "sum8_unscaled" in mut else 1.0)    # [n_blk]
        xs_ = xs[t].astype(np.float64)
        fd = (D * xs_[None]).reshape(rows, -1, 2).sum(axis=2)           # [rows, n_64]
        xm = (S * xs_).reshape(-1, 2).sum(axis=1)                        # [n_64]
        y[t] = (d * fd).sum(axis=1) + (m * xm[None]).sum(axis=1)
    return y


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("bits", [4, 6])
def test_embed_matches_closed_form(orc, bits):
    """Rows 0..39 (two full tiles and a half tile of 8 rows) of a 256-column
    matrix: value m + q d (a rounded product, a rounded sum), FWHT-64, signs."""
    rows, cols = 40, 256
    q, d16, m16 = random_codes(rows, cols, bits, 3 + bits)
    sb = M.sign_bits(cols, 9, "asym-embed")
    tiles, offs = build_tiles(q, d16, m16, bits)
    got = oracle_embed(orc, tiles, offs, sb, bits, cols, np.arange(rows))
    ref = embed_closed(q, d16, m16, sb)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-7), np.max(np.abs(got - ref))
    # planted layout mistakes in the tile move rows far off
    if bits == 6:
        tb, ob = build_tiles(q, d16, m16, bits, row_plane_swap=True)
        assert rel(oracle_embed(orc, tb, ob, sb, bits, cols, np.arange(rows)), ref) > 0.05
    tb, ob = build_tiles(q, m16, d16, bits)  # d and m exchanged
    assert rel(oracle_embed(orc, tb, ob, sb, bits, cols, np.arange(rows)), ref) > 0.05


@pytest.mark.parametrize("bits", [4, 6])
def test_gemv_matches_closed_form(orc, bits):
    """y for 3 tokens over 40 rows x 512 columns equals the float64 closed
    form to fp32 accumulation error; each planted mistake is far outside."""
    rows, cols = 40, 512
    q, d16, m16 = random_codes(rows, cols, bits, 11 + bits)
    sb = M.sign_bits(cols, 12, "asym-gemv")
    tiles, offs = build_tiles(q, d16, m16, bits)
    x = f32(np.random.default_rng(13).standard_normal((3, cols)))
    xq, xs, xm = oracle_prep(orc, x, sb)
    y = oracle_gemv(orc, tiles, offs, bits, rows, cols, xq, xs, xm)
    ref = gemv_closed(q, d16, m16, xq, xs)
    err = rel(y, ref)
    assert err < 1e-6, err
    muts = ["d_m_swapped", "halves_swapped", "sum8_unscaled"] + (["no_high_bits"] if bits == 6 else [])
    for mut in muts:
        assert rel(y, gemv_closed(q, d16, m16, xq, xs, mut=(mut,))) > 1e-2, mut
    if bits == 6:
        tb, ob = build_tiles(q, d16, m16, bits, row_plane_swap=True)
        assert rel(oracle_gemv(orc, tb, ob, bits, rows, cols, xq, xs, xm), ref) > 1e-2


@pytest.mark.parametrize("bits", [4, 6])
def test_gemv_m1_equals_m_rows_and_tile_range(orc, bits):
    """Every (row, token) is the same chain for M = 1 and M > 1 (the
    reference's M == 1 and slab branches agree, with no block skipped: a zero
    activation block still adds its terms); a tile range writes only its
    rows."""
    rows, cols = 48, 256
    q, d16, m16 = random_codes(rows, cols, bits, 21 + bits)
    sb = M.sign_bits(cols, 22, "asym-m")
    tiles, offs = build_tiles(q, d16, m16, bits)
    x = f32(np.random.default_rng(23).standard_normal((5, cols)))
    x[2, 64:96] = 0.0  # a zero block: scale 0, sum 0
    xq, xs, xm = oracle_prep(orc, x, sb)
    y5 = oracle_gemv(orc, tiles, offs, bits, rows, cols, xq, xs, xm)
    for i in range(5):
        y1 = oracle_gemv(orc, tiles, offs, bits, rows, cols, xq[i:i + 1], xs[i:i + 1], xm[i:i + 1])
        assert np.array_equal(y1[0].view(np.uint32), y5[i].view(np.uint32))
    part = oracle_gemv(orc, tiles, offs, bits, rows, cols, xq[:1], xs[:1], xm[:1], t0=1, t1=2, fill=9.0)
    assert (part[0, :16] == 9).all() and (part[0, 32:] == 9).all()
    assert np.array_equal(part[0, 16:32], y5[0, 16:32])


@pytest.mark.parametrize("bits,bound", [(4, 0.12), (6, 0.035)])
def test_packer_roundtrip_and_crc(orc, tools, bits, bound):
    """This repository's weighted-LSQ packer: tile CRCs verify, rows read
    back through the embedding recover N(0, 0.02) weights to 4 / 6-bit
    accuracy, no worse than a plain min/max code of the same width, and the
    GEMV of the packed tiles matches the dense product of those rows."""
    rows, cols = 72, 512
    W = M.random_normal(rows * cols, 0.02, 31, "asym-pack").reshape(rows, cols)
    sb = M.sign_bits(cols, 32, "asym-pack-s")
    blob, d = M.pack_matrix(W, sb, mode=13 if bits == 4 else 14)
    assert d.mode == (13 if bits == 4 else 14) and d.rows == rows and d.cols == cols
    tiles, offs, _ = M.desc_arrays(d)
    ok = np.zeros(d.n_tiles, np.uint8)
    assert tools.dpuf_qr_verify_tiles_ex(d.mode, d.n_tiles, cols, M.ptr(tiles), M.ptr(offs), M.ptr(ok)) == 0
    E = np.zeros((rows, cols), np.float32)
    ids = np.arange(rows, dtype=np.int32)
    orc.orc_embed_desc(C.byref(d), rows, M.ptr(ids), M.ptr(E))
    err = rel(E, W)
    assert err < bound, err
    # plain min/max code of the same width in the rotated domain
    Hm = hadamard64()
    s = signs_of(sb, cols)
    wr = ((W * s).reshape(rows, -1, 64) @ Hm.T)
    lo, hi = wr.min(axis=2, keepdims=True), wr.max(axis=2, keepdims=True)
    step = (hi - lo) / ((1 << bits) - 1)
    naive = lo + np.round((wr - lo) / step) * step
    naive_err = rel((naive @ Hm).reshape(rows, cols) * s, W)
    assert err <= naive_err * 1.02, (err, naive_err)
    x = f32(np.random.default_rng(33).standard_normal((2, cols)))
    xq, xs, xm = oracle_prep(orc, x, sb)
    y = oracle_gemv(orc, tiles, offs, bits, rows, cols, xq, xs, xm)
    xd = (xq.astype(np.float64).reshape(2, -1, 32) * xs[:, :, None]).reshape(2, cols)
    xd = (xd.reshape(2, -1, 64) @ Hm).reshape(2, cols) * s  # back from the rotated domain
    assert np.allclose(y, xd @ E.astype(np.float64).T, rtol=1e-4, atol=1e-5)


def test_hybrid_plan_modes(tools):
    """weight_plan 1 gives each matrix the mode of pack_dpuf.py:249-266 and
    signs of its own name."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=4, num_kv_heads=2, head_dim=64,
                 vocab_size=4096, tie_word_embeddings=0)
    m = M.Model.build(shape, max_seq_len=32, seed=41, weight_plan=1)
    assert m.tok.contents.mode == 13 and m.lm.contents.mode == 14
    want = {"w_q": 13, "w_k": 14, "w_v": 14, "w_gate": 13, "w_up": 13, "w_down": 14}
    for l in range(2):
        lw = m.layers[l]
        for k, v in want.items():
            assert getattr(lw, k).mode == v, (l, k)
        assert lw.w_o.mode == (14 if l % 2 == 0 else 13)
    sq = np.ctypeslib.as_array(C.cast(m.layers[0].w_q.sign_bits, C.POINTER(C.c_uint8)), (32,))
    sk = np.ctypeslib.as_array(C.cast(m.layers[0].w_k.sign_bits, C.POINTER(C.c_uint8)), (32,))
    assert not np.array_equal(sq, sk)
    m.close()
