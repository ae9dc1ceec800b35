"""GPU parity at the benchmark workloads' own shapes, and on every host path
the reference CLI drives, against the CPU oracle, through the C ABI.

Each test prints what it runs before it runs it.  Results are compared bit
for bit (logits, per-layer residuals, greedy ids): the engine reproduces the
reference's fp32 operation order, so equality is the bar, which is stricter
than the 1e-3 relative / 1e-4 absolute tolerance the workloads state.
"""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import model as M

pytestmark = pytest.mark.gpu


def log(*a):
    print(*a, flush=True)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def maxdiff(a, b):
    return float(np.max(np.abs(np.asarray(a, np.float64) - np.asarray(b, np.float64))))


def top_gap(x):
    t = np.sort(np.asarray(x, np.float64))[-2:]
    return float(t[1] - t[0])


class Pair:
    """A GPU engine and an oracle engine over the same model."""

    def __init__(self, eng, orc, model):
        self.eng, self.orc, self.m = eng, orc, model
        self.g = eng.dpuf_engine_create(*model.create_args())
        assert self.g, eng.dpuf_amd_last_error()
        self.o = orc.orc_engine_create(*model.create_args())
        assert self.o
        c = model.cfg.contents
        self.V, self.L, self.H = c.vocab_size, c.num_layers, c.hidden_size

    def forward(self, ids, pos0, only_last=1, embeds=None):
        n = len(ids) if ids is not None else embeds.shape[0]
        rows = 1 if only_last == 1 else n
        lg = np.zeros((rows, self.V), np.float32)
        lo = np.zeros((rows, self.V), np.float32)
        ip, ep = M.ptr(ids), M.ptr(embeds)
        rg = self.eng.dpuf_engine_forward_batch_ex(self.g, n, ip, pos0, ep, None, None, None, None, only_last,
                                                   M.ptr(lg) if only_last != 2 else None)
        ro = self.orc.orc_engine_forward(self.o, n, ip, pos0, ep, only_last, M.ptr(lo) if only_last != 2 else None)
        assert rg == 0 and ro == 0, (rg, ro, self.eng.dpuf_amd_last_error())
        return lg, lo

    def set_slot(self, s):
        assert self.eng.dpuf_engine_set_slot(self.g, s) == 0
        assert self.orc.orc_engine_set_slot(self.o, s) == 0

    def set_kv(self, layer, kvh, pos0, k, v):
        assert self.eng.dpuf_amd_engine_set_kv(self.g, layer, kvh, pos0, k.shape[0], M.ptr(k), M.ptr(v)) == 0
        assert self.orc.orc_engine_set_kv(self.o, layer, kvh, pos0, k.shape[0], M.ptr(k), M.ptr(v)) == 0

    def capture(self, cap):
        assert self.eng.dpuf_amd_engine_set_capture(self.g, cap) == 0
        self.orc.orc_engine_set_capture(self.o, cap)
        self.cap = cap

    def captured(self, rows):
        g = np.zeros(self.L * self.cap * self.H, np.float32)
        assert self.eng.dpuf_amd_engine_get_capture(self.g, M.ptr(g), g.size) == 0
        o = np.ctypeslib.as_array(C.cast(self.orc.orc_engine_get_capture(self.o), C.POINTER(C.c_float)),
                                  (self.L * self.cap * self.H,))
        return (g.reshape(self.L, self.cap, self.H)[:, :rows], o.reshape(self.L, self.cap, self.H)[:, :rows].copy())

    def close(self):
        self.eng.dpuf_engine_destroy(self.g)
        self.orc.orc_engine_destroy(self.o)


def greedy(p, first_logits_g, first_logits_o, pos, steps, what):
    """Greedy decode on both engines, each from its own argmax, comparing
    logits bit for bit and ids at every step; returns (ids, smallest
    top-1 / top-2 logit gap seen)."""
    tg, gap = [], float("inf")
    lg, lo = first_logits_g, first_logits_o
    for s in range(steps):
        a, b = int(np.argmax(lg[-1])), int(np.argmax(lo[-1]))
        assert a == b, (what, s, a, b)
        gap = min(gap, top_gap(lo[-1]))
        tg.append(a)
        lg, lo = p.forward(np.array([a], np.int32), pos + s)
        assert bits_equal(lg, lo), (what, s, maxdiff(lg, lo))
    return tg, gap


@pytest.mark.timeout(900)
def test_qwen3_8b_pp32_tg32_token_exact(eng, orc):
    """Qwen3-8B shape (36 layers, hidden 4096, 32 / 8 heads, FFN 12288,
    vocab 151936, untied LM head), N(0, 0.02) weights: a seeded 32-token
    prompt, then 32 greedy tokens.  Logits bit-identical at every step, ids
    identical."""
    log("building the Qwen3-8B-shape model (4.26 GB of packed weights)")
    m = M.Model.build(M.QWEN3_8B, max_seq_len=80, seed=1234)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(2024).integers(0, 151936, 32).astype(np.int32)
    log("8B pp32")
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    log("8B tg32")
    toks, gap = greedy(p, lg, lo, 32, 32, "8B")
    log("8B greedy ids", toks, "smallest top-1/top-2 gap", gap)
    p.close()


@pytest.mark.timeout(900)
def test_qwen3_8b_long_context_full_depth(eng, orc, monkeypatch):
    """The long-context workload at the Qwen3-8B shape and depth (36 layers,
    hidden 4096, 32 / 8 heads, FFN 12288, vocab 151936).  (a) pp512 of seeded
    ids on the M > 1 path with the down projection pruned to 224 of 256 tiles:
    the last row's logits bit-identical.  (b) Cache reset, a seeded N(0, 1)
    4096-position KV cache injected into all 36 x 8 heads of both engines,
    then 4 greedy one-token steps through the reference API (logits
    bit-identical, ids identical) and 2 through the captured-graph
    device-argmax entry (ids identical)."""
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "224")
    monkeypatch.delenv("DPUF_GEN_KEEP_TILES", raising=False)
    log("building the Qwen3-8B-shape model (4.26 GB of packed weights)")
    m = M.Model.build(M.QWEN3_8B, max_seq_len=4112, seed=4321)
    p = Pair(eng, orc, m)
    c = m.cfg.contents
    L, nkv, hd, V = c.num_layers, c.num_kv_heads, c.head_dim, c.vocab_size
    ids = np.random.default_rng(4322).integers(0, V, 512).astype(np.int32)
    log("8B pp512, keep 224 of 256 down tiles, 36 layers")
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    log("8B pp512 last-row top-1/top-2 gap", top_gap(lo[-1]))
    monkeypatch.delenv("DPUF_PREFILL_KEEP_TILES")
    eng.dpuf_engine_reset_slot(p.g, 0)
    orc.orc_engine_reset_slot(p.o, 0)
    log(f"injecting a 4096-position N(0, 1) KV cache into {L} x {nkv} heads")
    rng = np.random.default_rng(4323)
    for layer in range(L):
        for kvh in range(nkv):
            k = rng.standard_normal((4096, hd), dtype=np.float32)
            v = rng.standard_normal((4096, hd), dtype=np.float32)
            p.set_kv(layer, kvh, 0, k, v)
    tok = int(rng.integers(0, V))
    log("8B decode at position 4096 (36 layers, 4096 cached keys)")
    lg, lo = p.forward(np.array([tok], np.int32), 4096)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    toks, gap = greedy(p, lg, lo, 4097, 3, "8B 4096")
    log("8B long-context greedy ids", toks, "smallest top-1/top-2 gap", gap)
    tok = int(np.argmax(lo[-1]))
    out = C.c_int32(-1)
    for s in range(2):
        pos = 4100 + s
        log(f"8B graph decode with the device argmax at position {pos}")
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1,
                                                C.byref(out), None)
        assert rc == 0, eng.dpuf_amd_last_error()
        lo = np.zeros(V, np.float32)
        assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1, M.ptr(lo)) == 0
        assert out.value == orc.orc_argmax(M.ptr(lo), V)
        tok = out.value
    p.close()


def test_gqa4_long_context_injected_kv(eng, orc):
    """The Qwen3-8B attention geometry (32 Q / 8 KV heads: groups of 4,
    head_dim 128) on a small hidden size.  (1) Short context, the fused decode
    kernel: a 20-token prompt and 8 greedy steps.  (2) A 4096-position N(0, 1)
    KV cache injected into both engines, then 4 decode steps through the
    split attention (the long-context workload's kernels), then 3 more through
    the captured-graph device-argmax entry."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=32, num_kv_heads=8,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=4104, seed=71)
    p = Pair(eng, orc, m)
    log("G=4 short context: pp20 + 8 steps")
    ids = np.random.default_rng(72).integers(0, 4096, 20).astype(np.int32)
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo)
    greedy(p, lg, lo, 20, 8, "G4 short")
    log("G=4: injecting a 4096-position KV cache")
    rng = np.random.default_rng(73)
    for layer in range(2):
        for kvh in range(8):
            k = rng.standard_normal((4096, 128), dtype=np.float32)
            v = rng.standard_normal((4096, 128), dtype=np.float32)
            p.set_kv(layer, kvh, 0, k, v)
    lg, lo = p.forward(np.array([11], np.int32), 4096)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    toks, _ = greedy(p, lg, lo, 4097, 3, "G4 4096")
    tok = int(np.argmax(lo[-1]))
    out = C.c_int32(-1)
    for s in range(3):
        pos = 4100 + s
        log(f"G=4 graph decode at position {pos}")
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1,
                                                C.byref(out), None)
        assert rc == 0
        lo = np.zeros(4096, np.float32)
        assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1, M.ptr(lo)) == 0
        assert out.value == orc.orc_argmax(M.ptr(lo), 4096)
        tok = out.value
    p.close()


@pytest.mark.parametrize("nq,nkv,hd,ctx", [(16, 2, 128, 1000), (12, 2, 64, 700), (4, 2, 128, 2500)])
def test_one_token_long_context_groups(eng, orc, nq, nkv, hd, ctx):
    """One-token decode past the fused kernel's range with groups of 8, 6
    and 2 (the scores kernel's 8- and 2-row instances, the P.V kernel's 8-
    and 2-head ones): a ctx-position N(0, 1) KV cache injected into both
    engines, then 3 greedy steps, logits bit-identical."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=nq, num_kv_heads=nkv,
                 head_dim=hd, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=ctx + 8, seed=91)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(92)
    log(f"groups of {nq // nkv}, head dim {hd}: injecting {ctx} positions")
    for layer in range(2):
        for kvh in range(nkv):
            p.set_kv(layer, kvh, 0, rng.standard_normal((ctx, hd), dtype=np.float32),
                     rng.standard_normal((ctx, hd), dtype=np.float32))
    lg, lo = p.forward(np.array([5], np.int32), ctx)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, ctx + 1, 3, f"G{nq // nkv} ctx {ctx}")
    p.close()


WIDE, FALLBACK = 1, 3  # dpuf_amd_attn_path_count: one-token wide kernels, one-pair fallback


@pytest.mark.parametrize("nq,nkv,ctx", [(16, 2, 4096), (8, 2, 7500)])
def test_one_token_wide_path_beyond_lds_budget(eng, orc, nq, nkv, ctx):
    """One-token decode where the probability rows exceed the LDS budget of
    the split softmax / P.V kernel (groups of 8 at 4096 keys, groups of 4 at
    7500): the one-token kernels keep those rows in global memory, so eager
    steps take them (scores, softmax once per row, wide P.V), not the
    one-pair fallback; logits bit-identical."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=nq, num_kv_heads=nkv,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=ctx + 8, seed=95)
    p = Pair(eng, orc, m)
    eng.dpuf_amd_engine_set_graphs(p.g, 0)
    rng = np.random.default_rng(96)
    log(f"groups of {nq // nkv}: injecting {ctx} positions, eager decode")
    for layer in range(2):
        for kvh in range(nkv):
            p.set_kv(layer, kvh, 0, rng.standard_normal((ctx, 128), dtype=np.float32),
                     rng.standard_normal((ctx, 128), dtype=np.float32))
    w0, f0 = eng.dpuf_amd_attn_path_count(WIDE), eng.dpuf_amd_attn_path_count(FALLBACK)
    lg, lo = p.forward(np.array([5], np.int32), ctx)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    assert eng.dpuf_amd_attn_path_count(WIDE) - w0 == 2  # one launch set per layer
    assert eng.dpuf_amd_attn_path_count(FALLBACK) == f0
    greedy(p, lg, lo, ctx + 1, 2, f"G{nq // nkv} ctx {ctx} wide")
    p.close()


def test_graph_bucket_with_large_max_seq(eng, orc):
    """An engine created for 32768 positions decoding at about 300 keys
    through the captured-graph entry: the graph is captured for the key
    bucket of the position (512), not for max_seq, so its attention takes the
    one-token wide kernels as an eager step there would, not the one-pair
    fallback; ids equal the oracle's, and a step past the bucket (position
    520) captures the next one."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=8, num_kv_heads=2,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=32768, seed=97)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(98)
    for layer in range(2):
        for kvh in range(2):
            p.set_kv(layer, kvh, 0, rng.standard_normal((520, 128), dtype=np.float32),
                     rng.standard_normal((520, 128), dtype=np.float32))
    out = C.c_int32(-1)
    tok = 7
    for pos in (300, 301, 302, 520, 521):
        log(f"max_seq 32768: graph decode at position {pos}")
        w0, f0 = eng.dpuf_amd_attn_path_count(WIDE), eng.dpuf_amd_attn_path_count(FALLBACK)
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1,
                                                C.byref(out), None)
        assert rc == 0, eng.dpuf_amd_last_error()
        captured = eng.dpuf_amd_attn_path_count(WIDE) - w0
        assert captured == (2 if pos in (300, 520) else 0), (pos, captured)  # captured once per bucket
        assert eng.dpuf_amd_attn_path_count(FALLBACK) == f0
        lo = np.zeros(4096, np.float32)
        assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1, M.ptr(lo)) == 0
        assert out.value == orc.orc_argmax(M.ptr(lo), 4096)
        tok = out.value
    p.close()


def test_attention_beyond_split_lds_budget(eng, orc):
    """Groups of 4 with 7200 cached positions.  A two-token forward there:
    its rows of probabilities no longer fit the split kernels' LDS budget, so
    it takes the one-pair-per-workgroup kernel (k_attn); then one-token decode
    steps (the three-launch long-context path).  Logits bit-identical."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=1, num_q_heads=8, num_kv_heads=2,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=7240, seed=81)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(82)
    for kvh in range(2):
        p.set_kv(0, kvh, 0, rng.standard_normal((7200, 128), dtype=np.float32),
                 rng.standard_normal((7200, 128), dtype=np.float32))
    log("k_attn fallback: two tokens at position 7200")
    f0 = eng.dpuf_amd_attn_path_count(FALLBACK)
    lg, lo = p.forward(np.array([3, 4000], np.int32), 7200, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    assert eng.dpuf_amd_attn_path_count(FALLBACK) - f0 == 1
    greedy(p, lg, lo, 7202, 3, "after fallback")
    assert eng.dpuf_amd_attn_path_count(FALLBACK) - f0 == 1  # the one-token steps take the wide kernels
    p.close()


@pytest.mark.timeout(600)
def test_prefill_m512_8b_width_pruned(eng, orc, monkeypatch):
    """pp512 on the M > 1 path at the Qwen3-8B width (hidden 4096, FFN
    12288, 32 / 8 heads), two layers, down projection pruned to 224 of 256
    tiles: per-layer residual stream of all 512 rows and the last row's
    logits bit-identical; then 3 decode steps with the pruning off."""
    monkeypatch.setenv("DPUF_PREFILL_KEEP_TILES", "224")
    monkeypatch.delenv("DPUF_GEN_KEEP_TILES", raising=False)
    shape = dict(M.QWEN3_8B, num_layers=2, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=520, seed=91)
    p = Pair(eng, orc, m)
    p.capture(512)
    ids = np.random.default_rng(92).integers(0, 4096, 512).astype(np.int32)
    log("8B-width pp512, keep 224 of 256 down tiles")
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(512)
    assert bits_equal(cg, co), maxdiff(cg, co)
    assert np.all(co[:, :, 224 * 16:] != 0)  # the residual keeps its earlier values in pruned rows
    p.capture(0)
    greedy(p, lg, lo, 512, 3, "after pp512")
    p.close()


@pytest.mark.timeout(600)
def test_prefill_chunks_8b_width(eng, orc, monkeypatch):
    """Prefill in two chunks at the Qwen3-8B width (two layers): 200 tokens
    (the fused gate+up GEMM on 8-wave workgroups, a ragged last 64-token
    tile), per-layer residuals of every row and the last row's logits
    bit-identical; then 56 tokens at position 200 (4-wave workgroups) with
    every row's logits bit-identical; then 2 decode steps."""
    monkeypatch.delenv("DPUF_PREFILL_KEEP_TILES", raising=False)
    monkeypatch.delenv("DPUF_GEN_KEEP_TILES", raising=False)
    shape = dict(M.QWEN3_8B, num_layers=2, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=272, seed=93)
    p = Pair(eng, orc, m)
    p.capture(200)
    ids = np.random.default_rng(94).integers(0, 4096, 256).astype(np.int32)
    log("8B-width prefill chunks of 200 and 56 tokens")
    lg, lo = p.forward(ids[:200], 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(200)
    assert bits_equal(cg, co), maxdiff(cg, co)
    p.capture(0)
    lg, lo = p.forward(ids[200:], 200, only_last=0)
    assert lg.shape == (56, 4096)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 256, 2, "after 200 + 56")
    p.close()


@pytest.mark.timeout(600)
def test_lm_head_zone_a_151936(eng, orc, monkeypatch):
    """The LM head at its real size (151936 x 4096, 9496 tiles) with no
    layers, hidden states fed through embeds_in: 150 seeded steps, about 70 %
    with a planted zone token, Zone-A early exit on (1424 zone tiles, margin
    0.8), then 30 steps with it off.  Logits bit-identical at every step, so
    argmax ids and exit decisions are too."""
    shape = dict(M.QWEN3_8B, num_layers=0, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=16, seed=101)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(102)
    n = 150
    planted = rng.random(n) < 0.7
    tstar = rng.integers(0, 1424 * 16, n).astype(np.int32)
    hs = rng.standard_normal((n, 4096), dtype=np.float32)
    rows = np.zeros((n, 4096), np.float32)
    d = m.tok.contents
    orc.orc_embed(n, 4096, M.ptr(tstar), d.tensor_base, d.tile_offsets, d.sign_bits, M.ptr(rows))
    hs[planted] += np.float32(8.0) * rows[planted]
    monkeypatch.setenv("DPUF_EARLY_TILES", "1424")
    monkeypatch.setenv("DPUF_EARLY_MARGIN", "0.8")
    exits0 = eng.dpuf_amd_engine_early_exit_count(p.g)
    for i in range(n):
        if i % 25 == 0:
            log(f"LM head early exit step {i}")
        lg, lo = p.forward(None, 0, embeds=np.ascontiguousarray(hs[i:i + 1]))
        assert bits_equal(lg, lo), (i, maxdiff(lg, lo))
    exits = eng.dpuf_amd_engine_early_exit_count(p.g) - exits0
    log(f"early exit fired on {exits} of {n} steps ({planted.sum()} planted)")
    assert 0.5 * n < exits < n
    monkeypatch.delenv("DPUF_EARLY_TILES")
    for i in range(30):
        lg, lo = p.forward(None, 0, embeds=np.ascontiguousarray(hs[i:i + 1]))
        assert bits_equal(lg, lo), (i, maxdiff(lg, lo))
    p.close()


TINY = dict(hidden_size=256, intermediate_size=512, num_layers=3, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)


def test_chunked_prefill_only_last_2(eng, orc):
    """The CLI's long-prompt pattern (dpuf-cli.c:2384-2395): a 512-token
    prompt as two 256-token chunks, the first with only_last_logits = 2 (KV
    only, logits NULL), the second with 1; then greedy decode past 192
    positions."""
    m = M.Model.build(TINY, max_seq_len=600, seed=111)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(112).integers(0, 4096, 512).astype(np.int32)
    log("chunk 1 of 2, only_last_logits = 2")
    p.forward(ids[:256], 0, only_last=2)
    log("chunk 2 of 2, only_last_logits = 1")
    lg, lo = p.forward(ids[256:], 256)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 512, 4, "after chunks")
    p.close()


def test_embeds_in_rows(eng, orc):
    """embeds_in rows replace the embedding where token_ids[m] < 0, and for
    every row when token_ids is NULL (dpuf_engine.c:1658-1672)."""
    m = M.Model.build(TINY, max_seq_len=64, seed=121)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(122)
    emb = rng.standard_normal((6, 256), dtype=np.float32) * np.float32(0.05)
    ids = np.array([5, -1, 1000, -1, 7, -1], np.int32)
    log("embeds_in mixed with ids")
    lg, lo = p.forward(ids, 0, only_last=0, embeds=emb)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    log("embeds_in only")
    lg, lo = p.forward(None, 6, only_last=0, embeds=emb[:3].copy())
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 9, 3, "after embeds")
    p.close()


def test_one_row_embeds_steps_replay_a_graph(eng, orc):
    """One-row steps alternate between an embeds_in row (token_ids NULL, and
    token id -1) and a token id; the hidden state travels through host
    memory the embedding kernel reads, so both kinds replay the one graph
    captured for their shape: the fused decode attention is enqueued once per
    layer (at the capture), not once per layer per step.  Logits bit-identical
    to the oracle at every step."""
    m = M.Model.build(TINY, max_seq_len=64, seed=123)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(124)
    lg, lo = p.forward(rng.integers(0, 4096, 5).astype(np.int32), 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    emb = rng.standard_normal((12, 256), dtype=np.float32) * np.float32(0.05)
    dec0 = eng.dpuf_amd_attn_path_count(4)
    for s in range(12):
        pos = 5 + s
        if s % 3 == 0:
            lg, lo = p.forward(None, pos, embeds=emb[s:s + 1].copy())
        elif s % 3 == 1:
            lg, lo = p.forward(np.array([-1], np.int32), pos, embeds=emb[s:s + 1].copy())
        else:
            lg, lo = p.forward(np.array([int(np.argmax(lo[-1]))], np.int32), pos)
        assert bits_equal(lg, lo), (s, maxdiff(lg, lo))
    launched = eng.dpuf_amd_attn_path_count(4) - dec0
    log(f"fused decode attention enqueued {launched} times over 12 steps of {TINY['num_layers']} layers")
    assert launched == TINY["num_layers"], launched
    p.close()


def test_unshared_projection_signs(eng, orc):
    """Q, K, V with three different sign vectors (three activation preps,
    dpuf_engine.c:1760-1777) and gate / up with two, in every layer."""
    m = M.Model.build(TINY, max_seq_len=64, seed=131)
    rng = np.random.default_rng(132)
    for l in range(TINY["num_layers"]):
        lw = m.layers[l]
        for name in ("w_k", "w_v", "w_up"):
            d = getattr(lw, name)
            sb = np.ctypeslib.as_array(C.cast(d.sign_bits, C.POINTER(C.c_uint8)), (d.cols // 8,))
            sb[:] = rng.integers(0, 256, d.cols // 8)
    p = Pair(eng, orc, m)
    ids = rng.integers(0, 4096, 7).astype(np.int32)
    log("unshared signs: prefill 7 + 5 steps")
    lg, lo = p.forward(ids, 0, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 7, 5, "unshared")
    p.close()


def test_prefix_freeze_apply_reset(eng, orc):
    """Prefix cache (dpuf_engine.c:1438-1600) on both engines in lockstep: a
    12-token prompt on slot 0; positions [0, 8) frozen as prefix 2 and applied
    to slot 5; the rest of the prompt and 3 greedy steps on slot 5; slot 0
    continues on its own; after reset_slot(5) the same call on slot 5 sees
    zeros in positions [0, 8)."""
    m = M.Model.build(TINY, max_seq_len=64, seed=141)
    p = Pair(eng, orc, m)
    ids = np.random.default_rng(142).integers(0, 4096, 12).astype(np.int32)
    lg, lo = p.forward(ids, 0, only_last=0)
    assert bits_equal(lg, lo)
    assert eng.dpuf_engine_freeze_prefix(p.g, 2, 8) == 1 and orc.orc_engine_freeze_prefix(p.o, 2, 8) == 1
    assert eng.dpuf_engine_get_prefix_len(p.g, 2) == 8
    assert eng.dpuf_engine_apply_prefix(p.g, 5, 2) == 8 and orc.orc_engine_apply_prefix(p.o, 5, 2) == 8
    p.set_slot(5)
    assert eng.dpuf_engine_get_slot(p.g) == 5
    lg5, lo5 = p.forward(ids[8:], 8, only_last=0)
    assert bits_equal(lg5, lo5) and bits_equal(lg5, lg[8:])
    greedy(p, lg5, lo5, 12, 3, "slot 5")
    p.set_slot(0)
    greedy(p, lg, lo, 12, 2, "slot 0")
    eng.dpuf_engine_reset_slot(p.g, 5)
    orc.orc_engine_reset_slot(p.o, 5)
    p.set_slot(5)
    lr, lor = p.forward(ids[8:], 8, only_last=0)
    assert bits_equal(lr, lor) and not bits_equal(lr, lg5)
    assert eng.dpuf_engine_slot_memory(p.g) == 2 * 3 * 2 * 64 * 64 * 4
    p.close()


def test_few_row_steps_8b_width(eng, orc):
    """Steps of 2..16 rows at the Qwen3-8B width (hidden 4096, FFN 12288,
    two layers), whose Q/K/V and gate/up projections take the few-token
    GEMM: prefill chunks of 12 (16 staged tokens) and 5 rows (fragment
    pairs) with per-layer residuals, slot prompts of 3, 8, 5 and 2 rows
    (gate, up and the SwiGLU + down-input prep in one launch at 2..8 rows),
    then four sessions decoded together for 3 steps; every row
    bit-identical to the oracle."""
    shape = dict(M.QWEN3_8B, num_layers=2, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=64, seed=161)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(162)
    p.capture(16)
    ids = rng.integers(0, 4096, 17).astype(np.int32)
    log("8B-width prefill chunk of 12 rows")
    lg, lo = p.forward(ids[:12], 0, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(12)
    assert bits_equal(cg, co), maxdiff(cg, co)
    log("8B-width prefill chunk of 5 rows at position 12")
    lg, lo = p.forward(ids[12:], 12, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(5)
    assert bits_equal(cg, co), maxdiff(cg, co)
    p.capture(0)
    slots = np.array([1, 4, 6, 7], np.int32)
    toks, pos = [], []
    for s, n in zip(slots, (3, 8, 5, 2)):
        p.set_slot(int(s))
        lg, lo = p.forward(rng.integers(0, 4096, n).astype(np.int32), 0)
        assert bits_equal(lg, lo)
        toks.append(int(np.argmax(lo[0])))
        pos.append(n)
    for step in range(3):
        log(f"8B-width four-session step {step}")
        lg = np.zeros((len(slots), 4096), np.float32)
        got = np.full(len(slots), -1, np.int32)
        rc = eng.dpuf_amd_engine_forward_slots(p.g, len(slots), M.ptr(slots), M.ptr(np.array(toks, np.int32)),
                                              M.ptr(np.array(pos, np.int32)), M.ptr(lg), M.ptr(got))
        assert rc == 0, rc
        for i, s in enumerate(slots):
            assert orc.orc_engine_set_slot(p.o, int(s)) == 0
            lo = np.zeros(4096, np.float32)
            assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([toks[i]], np.int32)), pos[i], None, 1,
                                          M.ptr(lo)) == 0
            assert bits_equal(lg[i], lo), (step, i, maxdiff(lg[i], lo))
            assert got[i] == orc.orc_argmax(M.ptr(lo), 4096)
            toks[i] = int(got[i])
            pos[i] += 1
    p.close()


def test_few_row_swiglu_capped_workgroups_8b_width(eng, orc):
    """Gate, up and the SwiGLU + down-input prep in one few-token launch with
    its workgroups capped at 40 of the 192 it would take, so each walks 4 or
    5 of the down input's 64-blocks and reuses its LDS tile across rounds:
    prompts of 8 and 2 rows at the Qwen3-8B width (one layer), every row's
    logits bit-identical to the oracle."""
    shape = dict(M.QWEN3_8B, num_layers=1, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=32, seed=171)
    p = Pair(eng, orc, m)
    rng = np.random.default_rng(172)
    eng.dpuf_amd_set_gemv_max_workgroups(40)
    try:
        for s, n in ((2, 8), (3, 2)):
            log(f"capped few-token SwiGLU launch: {n}-row prompt in slot {s}")
            p.set_slot(s)
            lg, lo = p.forward(rng.integers(0, 4096, n).astype(np.int32), 0, only_last=0)
            assert bits_equal(lg, lo), (n, maxdiff(lg, lo))
    finally:
        eng.dpuf_amd_set_gemv_max_workgroups(0)
        p.close()


def test_multi_session_8b_attention_geometry(eng, orc):
    """dpuf_amd_engine_forward_slots with groups of 4 and head_dim 128 (two
    decode-attention workgroups per KV head, the second of which stores no
    KV) and an FFN of 4160 (the down projection's K > 4096 takes the
    one-fragment-per-workgroup K-split GEMM): three sessions, 4 steps, every
    row bit-identical to the oracle decoding that slot alone."""
    shape = dict(hidden_size=256, intermediate_size=4160, num_layers=2, num_q_heads=8, num_kv_heads=2,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    m = M.Model.build(shape, max_seq_len=64, seed=151)
    p = Pair(eng, orc, m)
    slots = np.array([2, 0, 7], np.int32)
    rng = np.random.default_rng(152)
    toks, pos = [], []
    for s, n in zip(slots, (6, 11, 4)):
        p.set_slot(int(s))
        lg, lo = p.forward(rng.integers(0, 4096, n).astype(np.int32), 0)
        assert bits_equal(lg, lo)
        toks.append(int(np.argmax(lo[0])))
        pos.append(n)
    for step in range(4):
        log(f"multi-session step {step}")
        lg = np.zeros((3, 4096), np.float32)
        got = np.full(3, -1, np.int32)
        rc = eng.dpuf_amd_engine_forward_slots(p.g, 3, M.ptr(slots), M.ptr(np.array(toks, np.int32)),
                                              M.ptr(np.array(pos, np.int32)), M.ptr(lg), M.ptr(got))
        assert rc == 0, rc
        for i, s in enumerate(slots):
            assert orc.orc_engine_set_slot(p.o, int(s)) == 0
            lo = np.zeros(4096, np.float32)
            assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([toks[i]], np.int32)), pos[i], None, 1,
                                          M.ptr(lo)) == 0
            assert bits_equal(lg[i], lo), (step, i, maxdiff(lg[i], lo))
            assert got[i] == orc.orc_argmax(M.ptr(lo), 4096)
            toks[i] = int(got[i])
            pos[i] += 1
    p.close()
