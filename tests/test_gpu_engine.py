"""End-to-end parity of the GPU engine (C ABI) against the CPU oracle."""
import numpy as np
import pytest

from dpuf_amd import model as M

pytestmark = pytest.mark.gpu

TINY = dict(hidden_size=256, intermediate_size=512, num_layers=3, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)


def _bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def _close(a, b, rtol=1e-3, atol=1e-4):
    return np.allclose(a, b, rtol=rtol, atol=atol)


class Pair:
    """A GPU engine and an oracle engine over the same model."""

    def __init__(self, eng, orc, model, cfg=None):
        self.eng, self.orc, self.m = eng, orc, model
        self.g = eng.dpuf_engine_create(*model.create_args(cfg))
        assert self.g, eng.dpuf_amd_last_error()
        self.o = orc.orc_engine_create(*model.create_args(cfg))
        assert self.o
        self.V = model.cfg.contents.vocab_size

    def forward(self, ids, pos0, only_last=1, embeds=None):
        n = len(ids) if ids is not None else embeds.shape[0]
        rows = 1 if only_last == 1 else n
        lg = np.zeros((rows, self.V), np.float32)
        lo = np.zeros((rows, self.V), np.float32)
        ip = M.ptr(ids) if ids is not None else None
        ep = M.ptr(embeds) if embeds is not None else None
        rg = self.eng.dpuf_engine_forward_batch_ex(self.g, n, ip, pos0, ep, None, None, None, None, only_last,
                                                   M.ptr(lg) if only_last != 2 else None)
        ro = self.orc.orc_engine_forward(self.o, n, ip, pos0, ep, only_last, M.ptr(lo) if only_last != 2 else None)
        assert rg == 0 and ro == 0, (rg, ro)
        return lg, lo

    def close(self):
        self.eng.dpuf_engine_destroy(self.g)
        self.orc.orc_engine_destroy(self.o)


@pytest.fixture(scope="module")
def tiny():
    return M.Model.build(TINY, max_seq_len=96, seed=5)


@pytest.mark.parametrize("cap", [0, 3])
def test_tiny_prefill_decode_bit_exact(eng, orc, tiny, cap):
    """cap 3 runs every M = 1 GEMV (QKV, O, gate/up, down, LM head) with three
    workgroups, each walking many groups."""
    eng.dpuf_amd_set_gemv_max_workgroups(cap)
    try:
        _prefill_decode(eng, orc, tiny)
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)


def test_hidden_states_and_down_pruning(eng, orc, tiny, monkeypatch):
    """Per-layer residual stream (h + hn after every layer) captured on both
    engines, with the down projection pruned to 10 of 16 tiles in decode and
    12 in prefill: bit-identical after the prefill and after every decode
    step."""
    import ctypes as C
    monkeypatch.setenv("DPUF_GEN_KEEP_TILES", "10")
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "12")
    p = Pair(eng, orc, tiny)
    L, H, cap = TINY["num_layers"], TINY["hidden_size"], 8
    assert eng.dpuf_amd_engine_set_capture(p.g, cap) == 0
    orc.orc_engine_set_capture(p.o, cap)

    def check(rows, what):
        g = np.zeros(L * cap * H, np.float32)
        assert eng.dpuf_amd_engine_get_capture(p.g, M.ptr(g), g.size) == 0
        o = np.ctypeslib.as_array(C.cast(orc.orc_engine_get_capture(p.o), C.POINTER(C.c_float)), (L * cap * H,))
        g = g.reshape(L, cap, H)[:, :rows]
        o = o.reshape(L, cap, H)[:, :rows]
        assert _bits_equal(g, o), (what, np.max(np.abs(g - o)))

    try:
        ids = np.random.default_rng(4).integers(0, 4096, 7).astype(np.int32)
        lg, lo = p.forward(ids, 0, only_last=0)
        assert _bits_equal(lg, lo)
        check(7, "prefill")
        tok = int(np.argmax(lo[-1]))
        for step in range(6):
            lg, lo = p.forward(np.array([tok], np.int32), 7 + step)
            assert _bits_equal(lg, lo), step
            check(1, f"decode step {step}")
            tok = int(np.argmax(lo[0]))
    finally:
        eng.dpuf_amd_engine_set_capture(p.g, 0)
        p.close()


def _prefill_decode(eng, orc, tiny):
    p = Pair(eng, orc, tiny)
    ids = np.random.default_rng(1).integers(0, 4096, 13).astype(np.int32)
    lg, lo = p.forward(ids, 0, only_last=0)
    assert _bits_equal(lg, lo), np.max(np.abs(lg - lo))
    tok = int(np.argmax(lo[-1]))
    for step in range(12):
        lg, lo = p.forward(np.array([tok], np.int32), 13 + step)
        assert _bits_equal(lg, lo), (step, np.max(np.abs(lg - lo)))
        tok = int(np.argmax(lo[0]))
    p.close()


def test_argmax_entry_and_graph(eng, orc, tiny):
    p = Pair(eng, orc, tiny)
    ids = np.random.default_rng(2).integers(0, 4096, 5).astype(np.int32)
    lg, lo = p.forward(ids, 0)
    tok = int(np.argmax(lo[0]))
    import ctypes as C
    out = C.c_int32(-1)
    for step in range(6):
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), 5 + step, None, 1,
                                                C.byref(out), None)
        assert rc == 0
        lo = np.zeros(4096, np.float32)
        orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), 5 + step, None, 1, M.ptr(lo))
        assert out.value == orc.orc_argmax(M.ptr(lo), 4096)
        tok = out.value
    p.close()


def test_graph_replay_switch(eng, orc):
    """Reference-API decode at 0.6B widths (2 layers, 8 kv heads of 4 query
    heads, hidden 1024): graph replay with the attention launch's cache
    warm-up (on by default), then every kernel enqueued
    (dpuf_amd_engine_set_graphs 0), then replay again; every step bit-equal
    to the oracle."""
    shape = dict(M.QWEN3_0_6B, num_layers=2, num_q_heads=32, vocab_size=8192)
    m = M.Model.build(shape, max_seq_len=64, seed=77)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(3).integers(0, 8192, 7).astype(np.int32)
    lg, lo = p.forward(ids, 0)
    assert _bits_equal(lg, lo)
    tok = int(np.argmax(lo[0]))
    for step in range(9):
        if step == 3:
            eng.dpuf_amd_engine_set_graphs(p.g, 0)
        if step == 6:
            eng.dpuf_amd_engine_set_graphs(p.g, 1)
        lg, lo = p.forward(np.array([tok], np.int32), 7 + step)
        assert _bits_equal(lg, lo), step
        tok = int(np.argmax(lo[0]))
    p.close()


def test_qwen3_06b_token_exact(eng, orc):
    """Qwen3-0.6B shape, random-init: 32-token prompt + 32 greedy tokens."""
    m = M.Model.build(M.QWEN3_0_6B, max_seq_len=80, seed=1234)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(2024).integers(0, 151936, 32).astype(np.int32)
    print("0.6B pp32", flush=True)
    lg, lo = p.forward(ids, 0)
    assert _close(lg, lo)
    tg, to = [], []
    tok_g, tok_o = int(np.argmax(lg[0])), int(np.argmax(lo[0]))
    exact = _bits_equal(lg, lo)
    for step in range(32):
        tg.append(tok_g)
        to.append(tok_o)
        lg, lo = p.forward(np.array([tok_o], np.int32), 32 + step)
        assert _close(lg, lo), step
        exact = exact and _bits_equal(lg, lo)
        tok_g, tok_o = int(np.argmax(lg[0])), int(np.argmax(lo[0]))
    print("greedy", tg, "bit-exact logits:", exact)
    assert tg == to
    assert exact
    p.close()


@pytest.mark.parametrize("cap", [0, 3])
def test_lm_early_exit(eng, orc, monkeypatch, cap):
    """Zone-A early exit of the LM head (more than 2048 tiles): with a tiny
    margin the zone's top-2 test fires and the rest of the vocabulary reads
    -1e9; with a huge margin it never fires and the full head runs.  Logits
    bit-identical to the oracle in both cases, at the default launch and with
    the GEMV workgroups capped (flag-gated launch walking many groups)."""
    shape = dict(TINY, vocab_size=40960)
    m = M.Model.build(shape, max_seq_len=32, seed=9)
    p = Pair(eng, orc, m)
    eng.dpuf_amd_set_gemv_max_workgroups(cap)
    try:
        ids = np.random.default_rng(3).integers(0, 40960, 6).astype(np.int32)
        monkeypatch.delenv("DPUF_EARLY_TILES", raising=False)
        lg, lo = p.forward(ids, 0)
        assert _bits_equal(lg, lo)
        tok = int(np.argmax(lo[0]))
        monkeypatch.setenv("DPUF_EARLY_TILES", "300")
        for step, margin in enumerate(["1e-7", "1e9", "1e-7"]):
            monkeypatch.setenv("DPUF_EARLY_MARGIN", margin)
            before = eng.dpuf_amd_engine_early_exit_count(p.g)
            lg, lo = p.forward(np.array([tok], np.int32), 6 + step)
            fired = eng.dpuf_amd_engine_early_exit_count(p.g) - before
            print(f"early exit cap={cap} margin={margin} fired={fired}", flush=True)
            assert _bits_equal(lg, lo), (margin, np.max(np.abs(lg - lo)))
            if margin == "1e9":
                assert fired == 0 and np.all(lo[0, 300 * 16:] > -1e8)
            else:
                assert fired == 1 and np.all(lo[0, 300 * 16:] == -1e9)
            tok = int(np.argmax(lo[0]))
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)
        p.close()


@pytest.mark.parametrize("heads", [(4, 2), (6, 2)])
def test_long_context_split_attention(eng, orc, heads):
    """Prefill in two chunks (M > 1 at pos0 0 and pos0 > 0) and decode past
    192 keys, where decode switches to the split attention kernels; also the
    captured-graph decode at that length.  (6, 2) heads give groups of three,
    so the third head takes the reference's single-head path.  Logits
    bit-identical to the oracle throughout."""
    nq, nkv = heads
    shape = dict(TINY, num_q_heads=nq, num_kv_heads=nkv)
    m = M.Model.build(shape, max_seq_len=320, seed=11)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(7)
    ids = rng.integers(0, 4096, 260).astype(np.int32)
    print(f"split attention heads={heads}: prefill 160 + 100", flush=True)
    lg, lo = p.forward(ids[:160], 0, only_last=0)
    assert _bits_equal(lg, lo), np.max(np.abs(lg - lo))
    lg, lo = p.forward(ids[160:], 160, only_last=0)
    assert _bits_equal(lg, lo), np.max(np.abs(lg - lo))
    tok = int(np.argmax(lo[-1]))
    for step in range(4):
        lg, lo = p.forward(np.array([tok], np.int32), 260 + step)
        assert _bits_equal(lg, lo), (step, np.max(np.abs(lg - lo)))
        tok = int(np.argmax(lo[0]))
    import ctypes as C
    out = C.c_int32(-1)
    for step in range(4, 8):
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), 260 + step, None, 1,
                                                C.byref(out), None)
        assert rc == 0
        lo = np.zeros(4096, np.float32)
        orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), 260 + step, None, 1, M.ptr(lo))
        assert out.value == orc.orc_argmax(M.ptr(lo), 4096)
        tok = out.value
    p.close()


def test_multi_session_decode(eng, orc, tiny):
    """Three sessions (KV slots 1, 4, 6) prefilled with prompts of different
    lengths, then four steps of one next token each through
    dpuf_amd_engine_forward_slots: every row's logits and greedy id equal the
    oracle decoding that slot on its own; a repeated slot is refused."""
    p = Pair(eng, orc, tiny)
    V = p.V
    slots = np.array([1, 4, 6], np.int32)
    rng = np.random.default_rng(17)
    toks, pos = [], []
    for s, n in zip(slots, (5, 9, 3)):
        assert eng.dpuf_engine_set_slot(p.g, int(s)) == 0
        assert orc.orc_engine_set_slot(p.o, int(s)) == 0
        lg, lo = p.forward(rng.integers(0, V, n).astype(np.int32), 0)
        assert _bits_equal(lg, lo)
        toks.append(int(np.argmax(lo[0])))
        pos.append(n)
    try:
        for step in range(4):
            lg = np.zeros((3, V), np.float32)
            ids = np.full(3, -1, np.int32)
            rc = eng.dpuf_amd_engine_forward_slots(p.g, 3, M.ptr(slots), M.ptr(np.array(toks, np.int32)),
                                                  M.ptr(np.array(pos, np.int32)), M.ptr(lg), M.ptr(ids))
            assert rc == 0, rc
            for i, s in enumerate(slots):
                assert orc.orc_engine_set_slot(p.o, int(s)) == 0
                lo = np.zeros(V, np.float32)
                orc.orc_engine_forward(p.o, 1, M.ptr(np.array([toks[i]], np.int32)), pos[i], None, 1, M.ptr(lo))
                assert _bits_equal(lg[i], lo), (step, i, np.max(np.abs(lg[i] - lo)))
                assert ids[i] == orc.orc_argmax(M.ptr(lo), V), (step, i)
                toks[i] = int(ids[i])
                pos[i] += 1
        dup = np.array([1, 1], np.int32)
        assert eng.dpuf_amd_engine_forward_slots(p.g, 2, M.ptr(dup), M.ptr(np.array(toks[:2], np.int32)),
                                                M.ptr(np.array(pos[:2], np.int32)), None, M.ptr(ids)) == -1
    finally:
        p.close()


def test_producer_fed_launches_two_engines_and_reruns(eng, orc):
    """One-row steps whose down projection (and, past the fused attention's
    range, O projection) prep their own input in producer workgroups of the
    same launch, signalled by flags that take a per-call serial: two engines
    stepped alternately (each with its own flags and serial), graph replays
    and the same positions run again after a cache reset, every step's
    logits bit-identical to the oracle."""
    shape = dict(TINY, num_layers=2)
    m = M.Model.build(shape, max_seq_len=260, seed=17)
    a, b = Pair(eng, orc, m), Pair(eng, orc, m)
    rng = np.random.default_rng(18)
    prompt = rng.integers(0, 4096, 200).astype(np.int32)
    for rnd in range(2):
        print(f"producer-fed: round {rnd}, prefill 200 on both engines", flush=True)
        for p in (a, b):
            eng.dpuf_engine_reset_cache(p.g)
            orc.orc_engine_reset_slot(p.o, 0)
            lg, lo = p.forward(prompt, 0)
            assert _bits_equal(lg, lo)
        toks = {id(a): int(np.argmax(lo[0])), id(b): int(np.argmax(lo[0]))}
        for step in range(6):
            for p in (a, b):  # alternate: each engine's flags hold the other's serials' neighbours
                lg, lo = p.forward(np.array([toks[id(p)]], np.int32), 200 + step)
                assert _bits_equal(lg, lo), (rnd, step, float(np.max(np.abs(lg - lo))))
                toks[id(p)] = int(np.argmax(lo[0]))
    a.close()
    b.close()
