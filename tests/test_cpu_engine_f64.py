"""Pins the oracle's engine composition (oracle/oracle.c orc_engine_forward,
restating dpuf_engine.c:1625-2170) against a float64 Qwen3 decoder written
from the mathematics (tests/f64_model.py).

The oracle quantises every GEMV input to int8 per 32-block, the float64 model
does not, so the two agree to the activation-quantisation noise (about 1 %
relative L2 on these shapes; the bound is 3 %).  Each mistake a restatement
could plausibly make -- a wrong GQA head map, a dropped QK-norm, RoPE on the
wrong pairs or with the wrong sign, an off-by-one causal length, a missing
residual, gate and up swapped, pruned rows left unzeroed, no dead zone, a wrong
early-exit fill -- is planted in the float64 model and must move it at least
5 % away from the oracle, so the bound cannot pass a restatement that has it.
CPU only.
"""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import model as M
from f64_model import F64Model

BOUND = 0.03      # oracle vs float64, relative L2 (activation quantisation noise)
CAUGHT = 0.05     # every planted mistake moves the float64 model at least this far

TINY = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)
MUTATIONS = ["gqa_modulo", "no_qk_norm", "rope_interleaved", "rope_sign", "causal_off_by_one", "no_attn_residual",
             "swiglu_swapped", "prune_unzeroed"]


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def randomise_norms(m, seed):
    """Norm weights U(0.5, 1.5) instead of the packer's 1.0, so a norm
    applied to the wrong index or not at all shows."""
    rng = np.random.default_rng(seed)
    c = m.cfg.contents
    for l in range(c.num_layers):
        lw = m.layers[l]
        for name, n in (("attn_norm", c.hidden_size), ("ffn_norm", c.hidden_size), ("attn_q_norm", c.head_dim),
                        ("attn_k_norm", c.head_dim)):
            a = np.ctypeslib.as_array(C.cast(getattr(lw, name), C.POINTER(C.c_float)), (n,))
            a[:] = rng.uniform(0.5, 1.5, n)
    a = np.ctypeslib.as_array(C.cast(m.out_norm, C.POINTER(C.c_float)), (c.hidden_size,))
    a[:] = rng.uniform(0.5, 1.5, c.hidden_size)


class OrcRun:
    """The oracle engine over a model, with per-layer residual capture."""

    def __init__(self, orc, m, cap=16):
        self.orc, self.m = orc, m
        c = m.cfg.contents
        self.L, self.H, self.V = c.num_layers, c.hidden_size, c.vocab_size
        self.h = orc.orc_engine_create(*m.create_args())
        assert self.h
        self.cap = cap
        orc.orc_engine_set_capture(self.h, cap)

    def forward(self, ids, pos0, only_last=0, embeds=None):
        n = len(ids) if ids is not None else embeds.shape[0]
        out = np.zeros((1 if only_last == 1 else n, self.V), np.float32)
        rc = self.orc.orc_engine_forward(self.h, n, M.ptr(ids), pos0, M.ptr(embeds), only_last, M.ptr(out))
        assert rc == 0
        capp = self.orc.orc_engine_get_capture(self.h)
        cap = np.ctypeslib.as_array(C.cast(capp, C.POINTER(C.c_float)), (self.L * self.cap * self.H,))
        return out, cap.reshape(self.L, self.cap, self.H)[:, :n].copy()

    def close(self):
        self.orc.orc_engine_destroy(self.h)


def _run_both(orc, shape, keep, mut_list, steps=3, prompt=9, seed=5, plan=0):
    m = M.Model.build(shape, max_seq_len=64, seed=seed, weight_plan=plan)
    randomise_norms(m, seed + 1)
    f = F64Model(orc, m)
    o = OrcRun(orc, m)
    V = shape["vocab_size"]
    ids = np.random.default_rng(seed + 2).integers(0, V, prompt).astype(np.int32)
    # the sequence: a prompt (M > 1), then greedy steps (M = 1) from the oracle's ids
    calls = []
    lo, capo = o.forward(ids, 0)
    calls.append((ids, 0, lo, capo))
    tok = int(np.argmax(lo[-1]))
    for s in range(steps):
        t = np.array([tok], np.int32)
        lo, capo = o.forward(t, prompt + s)
        calls.append((t, prompt + s, lo, capo))
        tok = int(np.argmax(lo[-1]))
    o.close()
    worst = {}
    for mut in [()] + [(x,) for x in mut_list]:
        f.reset()
        e = 0.0
        for ids_, pos0, lo, capo in calls:
            capf = []
            lf = f.forward(ids_, pos0, keep_tiles=keep, mut=mut, capture=capf)
            e = max(e, rel(lo, lf), max(rel(capo[l], capf[l]) for l in range(len(capf))))
        worst[mut] = e
    return worst


def test_oracle_engine_hybrid_matches_float64(orc, monkeypatch):
    """The same pinning for the had4p-hybrid plan (Modes 13 and 14 per
    pack_dpuf.py:249-266, separate signs for every matrix), group of 4, with
    the down projection pruned to 12 of 16 tiles."""
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "12")
    monkeypatch.setenv("DPUF_GEN_KEEP_TILES", "12")
    monkeypatch.delenv("DPUF_SWIGLU_DEADZONE", raising=False)
    w = _run_both(orc, dict(TINY, num_q_heads=8, num_kv_heads=2, tie_word_embeddings=0), 12, MUTATIONS, plan=1)
    print({k[0] if k else "exact": round(v, 4) for k, v in w.items()})
    assert w[()] < BOUND, w[()]
    for mut in MUTATIONS:
        assert w[(mut,)] > CAUGHT, (mut, w[(mut,)])


@pytest.mark.parametrize("heads", [(4, 2), (8, 2), (6, 2)])
def test_oracle_engine_matches_float64(orc, monkeypatch, heads):
    """Prefill of 9 tokens and 3 decode steps, down projection pruned to 12
    of 16 tiles: per-layer residual stream and logits of every call within
    BOUND of the float64 decoder; every planted mistake is caught.  Groups of
    2, 4 (the Qwen3-8B group) and 3 (a single trailing head)."""
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "12")
    monkeypatch.setenv("DPUF_GEN_KEEP_TILES", "12")
    monkeypatch.delenv("DPUF_SWIGLU_DEADZONE", raising=False)
    nq, nkv = heads
    w = _run_both(orc, dict(TINY, num_q_heads=nq, num_kv_heads=nkv), 12, MUTATIONS)
    print({k[0] if k else "exact": round(v, 4) for k, v in w.items()})
    assert w[()] < BOUND, w[()]
    for mut in MUTATIONS:
        assert w[(mut,)] > CAUGHT, (mut, w[(mut,)])


def test_oracle_deadzone_matches_float64(orc, monkeypatch):
    """With a dead zone of 0.03 (read at create, DPUF_SWIGLU_DEADZONE) a
    decoder without it is caught.  Values near the threshold land on either
    side in the two decoders, so the bound here is 3.5 % and a miss must move
    the result 7 %."""
    monkeypatch.setenv("DPUF_SWIGLU_DEADZONE", "0.03")
    m = M.Model.build(TINY, max_seq_len=64, seed=21)
    randomise_norms(m, 22)
    f = F64Model(orc, m)
    o = OrcRun(orc, m)
    ids = np.random.default_rng(23).integers(0, 4096, 9).astype(np.int32)
    lo, capo = o.forward(ids, 0)
    o.close()
    for mut, want in (((), "near"), (("no_deadzone",), "far")):
        f.reset()
        capf = []
        lf = f.forward(ids, 0, deadzone=0.03, mut=mut, capture=capf)
        e = max(rel(lo, lf), max(rel(capo[l], capf[l]) for l in range(len(capf))))
        assert (e < 0.035) if want == "near" else (e > 0.07), (mut, e)


def test_oracle_injected_kv_matches_float64(orc):
    """KV positions [0, 300) injected (N(0, 1), as the long-context workload
    does) into one layer of the oracle and the float64 decoder at the
    Qwen3-8B attention geometry (32 Q / 8 KV heads, head_dim 128), then two
    decode steps: logits within BOUND; a wrong GQA map is caught."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=1, num_q_heads=32, num_kv_heads=8,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=320, seed=31)
    randomise_norms(m, 32)
    f = F64Model(orc, m)
    o = OrcRun(orc, m)
    rng = np.random.default_rng(33)
    n = 300
    for kvh in range(8):
        k = rng.standard_normal((n, 128)).astype(np.float32)
        v = rng.standard_normal((n, 128)).astype(np.float32)
        assert orc.orc_engine_set_kv(o.h, 0, kvh, 0, n, M.ptr(k), M.ptr(v)) == 0
        f.set_kv(0, kvh, 0, k.astype(np.float64), v.astype(np.float64))
    toks = [7, 4095]
    outs = []
    for s, t in enumerate(toks):
        lo, _ = o.forward(np.array([t], np.int32), n + s)
        outs.append(lo)
    o.close()
    for mut, want in (((), "near"), (("gqa_modulo",), "far")):
        f.kc, f.vc = f.kc[:, :, :n].copy(), f.vc[:, :, :n].copy()
        e = 0.0
        for s, t in enumerate(toks):
            lf = f.forward(np.array([t], np.int32), n + s, mut=mut)
            e = max(e, rel(outs[s], lf))
        assert (e < BOUND) if want == "near" else (e > CAUGHT), (mut, e)


def test_oracle_early_exit_fill(orc, monkeypatch):
    """Zone-A early exit on an LM head of 2560 tiles, hidden states fed in
    (no layers): with a planted zone token the margin test fires and every
    logit past the zone is exactly -1e9 (a different fill is caught); zone
    logits within BOUND of the float64 head; without the plant the margin is
    not met and the full head runs."""
    shape = dict(TINY, num_layers=0, vocab_size=40960)
    m = M.Model.build(shape, max_seq_len=16, seed=41)
    randomise_norms(m, 42)
    f = F64Model(orc, m)
    o = OrcRun(orc, m)
    monkeypatch.setenv("DPUF_EARLY_TILES", "300")
    monkeypatch.setenv("DPUF_EARLY_MARGIN", "0.8")
    rng = np.random.default_rng(43)
    h = rng.standard_normal((1, 256)).astype(np.float32)
    planted = (h + 40.0 * f.E[1234].astype(np.float32)).astype(np.float32)
    for x, fires in ((planted, True), (h, False)):
        lo, _ = o.forward(None, 0, only_last=1, embeds=np.ascontiguousarray(x))
        lf = f.forward(None, 0, embeds=x, early=(300, 0.8))
        nz = 300 * 16
        assert rel(lo[0, :nz], lf[0, :nz]) < BOUND
        if fires:
            assert int(np.argmax(lo[0])) == 1234
            assert np.all(lo[0, nz:] == np.float32(-1e9)) and np.all(lf[0, nz:] == -1e9)
            lw = f.forward(None, 0, embeds=x, early=(300, 0.8), mut=("fill_wrong",))
            assert not np.all(lo[0, nz:] == lw[0, nz:])
        else:
            assert np.all(lo[0, nz:] > -1e8) and rel(lo[0], lf[0]) < BOUND
    o.close()


def test_oracle_prefix_freeze_apply_and_reset(orc):
    """Prefix cache of dpuf_engine.c:1438-1600 restated in the oracle: a
    12-token prompt on slot 0, its first 8 positions frozen as prefix 2 and
    applied to slot 5; running tokens 8..11 on slot 5 from position 8 gives
    the logits of rows 8..11 of the full prompt bit for bit, and the next
    greedy steps agree on both slots.  After reset_slot(5) the same call
    differs (the prefix was the only source of positions 0..7)."""
    m = M.Model.build(TINY, max_seq_len=64, seed=51)
    o = OrcRun(orc, m)
    ids = np.random.default_rng(52).integers(0, 4096, 12).astype(np.int32)
    full, _ = o.forward(ids, 0)
    assert orc.orc_engine_freeze_prefix(o.h, 2, 8) == 1
    assert orc.orc_engine_apply_prefix(o.h, 5, 2) == 8
    assert orc.orc_engine_set_slot(o.h, 5) == 0
    part, _ = o.forward(ids[8:], 8)
    assert np.array_equal(part.view(np.uint32), full[8:].view(np.uint32))
    tok = int(np.argmax(full[-1]))
    for s in range(3):
        assert orc.orc_engine_set_slot(o.h, 5) == 0
        a, _ = o.forward(np.array([tok], np.int32), 12 + s)
        assert orc.orc_engine_set_slot(o.h, 0) == 0
        b, _ = o.forward(np.array([tok], np.int32), 12 + s)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), s
        tok = int(np.argmax(a[-1]))
    orc.orc_engine_reset_slot(o.h, 5)
    assert orc.orc_engine_set_slot(o.h, 5) == 0
    again, _ = o.forward(ids[8:], 8)
    assert not np.array_equal(again, part)
    o.close()


def test_oracle_embeds_rows_replace_embedding(orc):
    """embeds_in rows stand in for ids < 0 (dpuf_engine.c:1658-1672): a row
    holding the embedding of id t gives the logits of id t bit for bit."""
    m = M.Model.build(TINY, max_seq_len=64, seed=61)
    f = F64Model(orc, m)
    o = OrcRun(orc, m)
    ids = np.array([5, 99, 1000, 7], np.int32)
    a, _ = o.forward(ids, 0)
    emb = np.zeros((4, 256), np.float32)
    orc.orc_embed(4, 256, M.ptr(ids), m.tok.contents.tensor_base, m.tok.contents.tile_offsets,
                  m.tok.contents.sign_bits, M.ptr(emb))
    assert np.allclose(emb, f.E[ids], atol=0)
    mixed = ids.copy()
    mixed[[1, 3]] = -1
    orc.orc_engine_reset_slot(o.h, 0)
    b, _ = o.forward(mixed, 0, embeds=emb)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    o.close()


# --------------------------------------------------------------------------- Q8 KV cache

def _q8(orc, x):
    n = x.size
    q = np.zeros(n, np.int8)
    s = np.zeros(n // 32, np.float32)
    orc.orc_quant_q8(n, M.ptr(np.ascontiguousarray(x, np.float32)), M.ptr(q), M.ptr(s))
    return q, s


def test_q8_quantisation_cases(orc):
    """quantize_vec_q8_blk32 (dpuf_engine.c:754-781): per 32-block scale
    amax / 127; the extreme value maps to +-127; an all-zero block gives q = 0;
    exact ties k + 1/2 round to even; |x - q * scale| <= scale / 2; the block
    boundaries are every 32 values."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(128).astype(np.float32)
    x[32:64] = 0.0
    x[70] = -9.0  # block 2's extreme, negative
    q, s = _q8(orc, x)
    for b in range(4):
        blk = x[32 * b:32 * b + 32]
        amax = np.float32(np.max(np.abs(blk)))
        assert s[b] == np.float32(amax / np.float32(127.0))
        if amax == 0:
            assert (q[32 * b:32 * b + 32] == 0).all()
            continue
        err = np.abs(blk.astype(np.float64) - q[32 * b:32 * b + 32].astype(np.float64) * s[b])
        assert err.max() <= s[b] / 2 * (1 + 1e-5)
    assert q[70] == -127 and q.min() >= -127
    # ties: amax 127 makes inv exactly 1, so x = k + 0.5 rounds to even
    t = np.zeros(32, np.float32)
    t[0] = 127.0
    t[1:6] = [0.5, 1.5, 2.5, -0.5, -3.5]
    q, s = _q8(orc, t)
    assert list(q[:6]) == [127, 0, 2, 2, 0, -4] and s[0] == np.float32(1.0)


@pytest.mark.parametrize("n,pair", [(1, False), (7, True), (9, False), (40, True)])
def test_q8_attention_float64(orc, n, pair):
    """gqa_attn_head_pair_q8 restated: softmax(q . k_deq / sqrt(hd)) v_deq in
    float64 over the dequantised int8 K/V to 1e-5 (both query paths, odd key
    counts that take the single-key tail)."""
    rng = np.random.default_rng(100 + n)
    hd = 128
    K = rng.standard_normal((n, hd)).astype(np.float32)
    V = rng.standard_normal((n, hd)).astype(np.float32)
    kq, ks = _q8(orc, K.ravel())
    vq, vs = _q8(orc, V.ravel())
    Kd = kq.reshape(n, hd).astype(np.float64) * np.repeat(ks.reshape(n, hd // 32), 32, axis=1)
    Vd = vq.reshape(n, hd).astype(np.float64) * np.repeat(vs.reshape(n, hd // 32), 32, axis=1)
    q0 = rng.standard_normal(hd).astype(np.float32)
    q1 = rng.standard_normal(hd).astype(np.float32) if pair else None
    sc0, sc1 = np.zeros(n, np.float32), np.zeros(n, np.float32)
    o0, o1 = np.zeros(hd, np.float32), np.zeros(hd, np.float32)
    orc.orc_attn_heads_q8(hd, n, C.c_float(1 / np.sqrt(hd)), M.ptr(kq), M.ptr(ks), M.ptr(vq), M.ptr(vs), M.ptr(q0),
                          M.ptr(q1), M.ptr(sc0), M.ptr(sc1), M.ptr(o0), M.ptr(o1) if pair else None)
    for q, o in ((q0, o0), (q1, o1)):
        if q is None:
            continue
        s = Kd @ q.astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(o, p @ Vd, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("heads", [(4, 2), (8, 2), (6, 2)])
def test_oracle_q8_engine_matches_float64(orc, heads):
    """kv_type 1 (the int8 KV cache, dpuf_engine.c:1191-1197, 1800-1806):
    prefill + 3 decode steps of the oracle within BOUND of the float64
    decoder holding the same int8 round trip of K and V; using a neighbouring
    block's scale is caught."""
    nq, nkv = heads
    m = M.Model.build(dict(TINY, num_q_heads=nq, num_kv_heads=nkv), max_seq_len=64, seed=7)
    randomise_norms(m, 8)
    cfg = M.abi.DpufModelConfig.from_buffer_copy(m.cfg.contents)
    cfg.kv_type = 1
    f = F64Model(orc, m)
    oh = orc.orc_engine_create(C.byref(cfg), m.layers, m.tok, m.lm, m.out_norm)
    assert oh
    ids = np.random.default_rng(9).integers(0, 4096, 9).astype(np.int32)
    calls = []
    lo = np.zeros((9, 4096), np.float32)
    assert orc.orc_engine_forward(oh, 9, M.ptr(ids), 0, None, 0, M.ptr(lo)) == 0
    calls.append((ids, 0, lo.copy()))
    tok = int(np.argmax(lo[-1]))
    for s in range(3):
        t = np.array([tok], np.int32)
        l1 = np.zeros((1, 4096), np.float32)
        assert orc.orc_engine_forward(oh, 1, M.ptr(t), 9 + s, None, 1, M.ptr(l1)) == 0
        calls.append((t, 9 + s, l1.copy()))
        tok = int(np.argmax(l1[-1]))
    orc.orc_engine_destroy(oh)
    errs = {}
    for mut in ((), ("q8_scale_shift",)):
        f.reset()
        errs[mut] = max(rel(lo_, f.forward(i_, p_, kv_q8=True, mut=mut)[-lo_.shape[0]:]) for i_, p_, lo_ in calls)
    print(errs)
    assert errs[()] < BOUND and errs[("q8_scale_shift",)] > CAUGHT


def test_oracle_q8_prefix_and_inject(orc):
    """With kv_type 1, freeze -> apply reproduces the prompt's logits bit
    for bit from the prefix position, and set_kv quantises injected rows as
    the store does: get_kv returns them dequantised within half a step."""
    m = M.Model.build(TINY, max_seq_len=64, seed=11)
    cfg = M.abi.DpufModelConfig.from_buffer_copy(m.cfg.contents)
    cfg.kv_type = 1
    oh = orc.orc_engine_create(C.byref(cfg), m.layers, m.tok, m.lm, m.out_norm)
    ids = np.random.default_rng(12).integers(0, 4096, 12).astype(np.int32)
    full = np.zeros((12, 4096), np.float32)
    assert orc.orc_engine_forward(oh, 12, M.ptr(ids), 0, None, 0, M.ptr(full)) == 0
    assert orc.orc_engine_freeze_prefix(oh, 1, 8) == 1
    assert orc.orc_engine_apply_prefix(oh, 3, 1) == 8
    assert orc.orc_engine_set_slot(oh, 3) == 0
    part = np.zeros((4, 4096), np.float32)
    assert orc.orc_engine_forward(oh, 4, M.ptr(ids[8:]), 8, None, 0, M.ptr(part)) == 0
    assert np.array_equal(part.view(np.uint32), full[8:].view(np.uint32))
    rng = np.random.default_rng(13)
    k = rng.standard_normal((5, 64)).astype(np.float32)
    v = rng.standard_normal((5, 64)).astype(np.float32)
    assert orc.orc_engine_set_kv(oh, 1, 1, 20, 5, M.ptr(k), M.ptr(v)) == 0
    kb, vb = np.zeros_like(k), np.zeros_like(v)
    assert orc.orc_engine_get_kv(oh, 1, 1, 20, 5, M.ptr(kb), M.ptr(vb)) == 0
    for a, b in ((k, kb), (v, vb)):
        step = np.max(np.abs(a.reshape(-1, 32)), axis=1) / 127
        assert np.all(np.abs(a - b).reshape(-1, 32) <= step[:, None] * 0.5 * (1 + 1e-5))
    orc.orc_engine_destroy(oh)
