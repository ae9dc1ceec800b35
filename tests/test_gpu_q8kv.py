"""The int8 KV cache (kv_type 1; reference dpuf_engine.c:579-781, 1182-1206,
1800-1806) on the GPU against the oracle's restatement: per-32-block int8 K
and V with fp32 scales, the quantising store after QK-norm and RoPE, and the
int8-cache attention.  Bit for bit, through the C ABI."""
import ctypes as C

import numpy as np
import pytest

from dpuf_amd import abi
from dpuf_amd import model as M
from test_gpu_configs import Pair, bits_equal, greedy, log, maxdiff

pytestmark = pytest.mark.gpu


def q8_model(shape, max_seq, seed):
    m = M.Model.build(shape, max_seq_len=max_seq, seed=seed)
    cfg = abi.DpufModelConfig.from_buffer_copy(m.cfg.contents)
    cfg.kv_type = 1
    return m, cfg


class Q8Pair(Pair):
    def __init__(self, eng, orc, model, cfg):
        self.eng, self.orc, self.m = eng, orc, model
        self.cfg = cfg
        self.g = eng.dpuf_engine_create(*model.create_args(cfg))
        assert self.g, eng.dpuf_amd_last_error()
        self.o = orc.orc_engine_create(*model.create_args(cfg))
        assert self.o
        self.V, self.L, self.H = cfg.vocab_size, cfg.num_layers, cfg.hidden_size


TINY = dict(hidden_size=256, intermediate_size=512, num_layers=3, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)


@pytest.mark.parametrize("heads,hd", [((4, 2), 64), ((6, 2), 64), ((8, 2), 128)])
def test_q8_prefill_decode_bit_exact(eng, orc, heads, hd):
    """Prefill of 13 tokens (M > 1) and 10 greedy steps (M = 1): logits and
    the per-layer residual stream bit-identical; groups of 2, 3 (the single
    trailing head) and 4; the slot memory is the int8 layout's."""
    nq, nkv = heads
    m, cfg = q8_model(dict(TINY, num_q_heads=nq, num_kv_heads=nkv, head_dim=hd), 64, 201)
    p = Q8Pair(eng, orc, m, cfg)
    p.capture(16)
    ids = np.random.default_rng(202).integers(0, 4096, 13).astype(np.int32)
    log(f"q8 kv heads={heads} hd={hd}: prefill 13")
    lg, lo = p.forward(ids, 0, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    cg, co = p.captured(13)
    assert bits_equal(cg, co), maxdiff(cg, co)
    greedy(p, lg, lo, 13, 10, "q8")
    rows = 3 * nkv * 64
    assert eng.dpuf_engine_slot_memory(p.g) == 2 * rows * hd + 2 * rows * (hd // 32) * 4
    p.close()


def test_q8_injected_context_and_graph(eng, orc):
    """300 N(0, 1) K/V positions injected through set_kv (quantised on both
    sides as the store does) at the Qwen3-8B attention geometry, then decode
    on the reference entry and on the captured-graph device-argmax entry;
    get_kv returns the dequantised rows of both engines bit for bit."""
    shape = dict(TINY, num_layers=2, num_q_heads=32, num_kv_heads=8, head_dim=128)
    m, cfg = q8_model(shape, 320, 211)
    p = Q8Pair(eng, orc, m, cfg)
    rng = np.random.default_rng(212)
    for layer in range(2):
        for kvh in range(8):
            p.set_kv(layer, kvh, 0, rng.standard_normal((300, 128), dtype=np.float32),
                     rng.standard_normal((300, 128), dtype=np.float32))
    kg, vg = np.zeros((300, 128), np.float32), np.zeros((300, 128), np.float32)
    ko, vo = kg.copy(), vg.copy()
    assert eng.dpuf_amd_engine_get_kv(p.g, 1, 5, 0, 300, M.ptr(kg), M.ptr(vg)) == 0
    assert orc.orc_engine_get_kv(p.o, 1, 5, 0, 300, M.ptr(ko), M.ptr(vo)) == 0
    assert bits_equal(kg, ko) and bits_equal(vg, vo)
    log("q8 kv: decode after 300 injected positions")
    lg, lo = p.forward(np.array([17], np.int32), 300)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 301, 3, "q8 inject")
    tok = int(np.argmax(lo[-1]))
    out = C.c_int32(-1)
    for s in range(3):
        pos = 304 + s
        rc = eng.dpuf_amd_engine_forward_argmax(p.g, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1,
                                                C.byref(out), None)
        assert rc == 0
        lo = np.zeros(4096, np.float32)
        assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([tok], np.int32)), pos, None, 1, M.ptr(lo)) == 0
        assert out.value == orc.orc_argmax(M.ptr(lo), 4096)
        tok = out.value
    p.close()


def test_q8_prefix_slots_and_refusals(eng, orc):
    """Prefix freeze / apply / reset and a second slot with the int8 cache,
    in lockstep with the oracle; then one multi-session step on the int8
    cache, its greedy id equal to the oracle's."""
    m, cfg = q8_model(TINY, 64, 221)
    p = Q8Pair(eng, orc, m, cfg)
    ids = np.random.default_rng(222).integers(0, 4096, 12).astype(np.int32)
    lg, lo = p.forward(ids, 0, only_last=0)
    assert bits_equal(lg, lo)
    assert eng.dpuf_engine_freeze_prefix(p.g, 1, 8) == 1 and orc.orc_engine_freeze_prefix(p.o, 1, 8) == 1
    assert eng.dpuf_engine_apply_prefix(p.g, 4, 1) == 8 and orc.orc_engine_apply_prefix(p.o, 4, 1) == 8
    p.set_slot(4)
    l4, o4 = p.forward(ids[8:], 8, only_last=0)
    assert bits_equal(l4, o4) and bits_equal(l4, lg[8:])
    greedy(p, l4, o4, 12, 3, "q8 slot 4")
    eng.dpuf_engine_reset_slot(p.g, 4)
    orc.orc_engine_reset_slot(p.o, 4)
    lr, lor = p.forward(ids[8:], 8, only_last=0)
    assert bits_equal(lr, lor)
    # the multi-session entry serves the int8 cache too: slot 4 at position 12
    got = np.zeros(1, np.int32)
    rc = eng.dpuf_amd_engine_forward_slots(p.g, 1, M.ptr(np.array([4], np.int32)), M.ptr(np.array([5], np.int32)),
                                          M.ptr(np.array([12], np.int32)), None, M.ptr(got))
    assert rc == 0, (rc, eng.dpuf_amd_last_error())
    assert orc.orc_engine_set_slot(p.o, 4) == 0
    lo = np.zeros(p.V, np.float32)
    assert orc.orc_engine_forward(p.o, 1, M.ptr(np.array([5], np.int32)), 12, None, 1, M.ptr(lo)) == 0
    assert got[0] == orc.orc_argmax(M.ptr(lo), p.V)
    p.close()


def test_q8_rows_beyond_lds(eng, orc):
    """7200 cached positions with groups of 4: a two-token forward's
    probability rows no longer fit the split kernel's LDS budget, so it takes
    the softmax-in-memory kernel (k_attn_q8); one-token steps after it take
    the split kernel again.  Bit-identical."""
    shape = dict(TINY, num_layers=1, num_q_heads=8, num_kv_heads=2, head_dim=128)
    m, cfg = q8_model(shape, 7240, 231)
    p = Q8Pair(eng, orc, m, cfg)
    rng = np.random.default_rng(232)
    for kvh in range(2):
        p.set_kv(0, kvh, 0, rng.standard_normal((7200, 128), dtype=np.float32),
                 rng.standard_normal((7200, 128), dtype=np.float32))
    log("q8 kv: two tokens at position 7200")
    lg, lo = p.forward(np.array([3, 4000], np.int32), 7200, only_last=0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 7202, 3, "q8 after 7200")
    p.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("nq", [32, 64])
def test_q8_4096_injected_keys(eng, orc, nq):
    """A 4096-position N(0, 1) KV cache injected into the int8 cache of both
    engines (8 KV heads, head_dim 128, groups of 4 and 8), then 3 decode steps
    through the one-token long-context kernels (softmax once per row, P.V
    chain waves fed W = p * v_scale and widened V by producer waves): logits
    bit for bit at every step."""
    shape = dict(TINY, num_layers=1, num_q_heads=nq, num_kv_heads=8, head_dim=128)
    m, cfg = q8_model(shape, 4104, 221)
    p = Q8Pair(eng, orc, m, cfg)
    rng = np.random.default_rng(222)
    log(f"q8 kv: injecting 4096 positions, groups of {nq // 8}")
    for kvh in range(8):
        p.set_kv(0, kvh, 0, rng.standard_normal((4096, 128), dtype=np.float32),
                 rng.standard_normal((4096, 128), dtype=np.float32))
    lg, lo = p.forward(np.array([23], np.int32), 4096)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 4097, 3, f"q8 4096 G{nq // 8}")
    p.close()


@pytest.mark.parametrize("nq,nkv,kv_type", [(8, 2, 0), (4, 2, 0), (16, 2, 0), (8, 2, 1), (4, 2, 1)])
def test_one_token_last_positions_unaligned_max_seq(eng, orc, nq, nkv, kv_type):
    """An engine created for 1029 positions (not a multiple of 4) decoding its
    last three positions, 1026 .. 1028, after 1026 injected keys, for groups
    of 4, 2 and 8 over the fp32 cache and groups of 4 and 2 over the int8
    cache: the one-token kernels read the probability rows' last keys one by
    one there (a 16-byte piece would run past the row), so the logits stay
    bit-identical up to the context's end."""
    shape = dict(TINY, num_layers=2, num_q_heads=nq, num_kv_heads=nkv, head_dim=128)
    m, cfg = q8_model(shape, 1029, 301)
    cfg.kv_type = kv_type
    p = Q8Pair(eng, orc, m, cfg)
    rng = np.random.default_rng(302)
    for layer in range(2):
        for kvh in range(nkv):
            p.set_kv(layer, kvh, 0, rng.standard_normal((1026, 128), dtype=np.float32),
                     rng.standard_normal((1026, 128), dtype=np.float32))
    log(f"max_seq 1029, groups of {nq // nkv}, kv_type {kv_type}: positions 1026 .. 1028")
    lg, lo = p.forward(np.array([9], np.int32), 1026)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 1027, 2, f"unaligned max_seq G{nq // nkv} kv{kv_type}")
    p.close()


@pytest.mark.parametrize("kv_type", [0, 1])
def test_multi_session_mixed_lengths(eng, orc, kv_type):
    """dpuf_amd_engine_forward_slots serving sessions of very different
    lengths in one pass, over the fp32 (kv_type 0) and int8 (kv_type 1)
    caches, at the Qwen3-8B attention geometry (groups of 4, head_dim 128):
    four sessions, one past 4096 keys (injected), one at 300, two short ones
    prefilled normally, passed in an order that mixes them; 3 steps, every row
    bit-identical to the oracle decoding that slot alone, ids too."""
    shape = dict(TINY, num_layers=2, num_q_heads=8, num_kv_heads=2, head_dim=128)
    m, cfg = q8_model(shape, 4200, 401)
    cfg.kv_type = kv_type
    p = Q8Pair(eng, orc, m, cfg)
    rng = np.random.default_rng(402)
    slots = np.array([5, 1, 6, 3], np.int32)
    lens = {5: 4100, 1: 9, 6: 300, 3: 40}
    toks, pos = [], []
    for s in slots:
        s = int(s)
        p.set_slot(s)
        n = lens[s]
        if n > 64:
            # an injected context, then one token through the normal path
            for layer in range(2):
                for kvh in range(2):
                    p.set_kv(layer, kvh, 0, rng.standard_normal((n - 1, 128), dtype=np.float32),
                             rng.standard_normal((n - 1, 128), dtype=np.float32))
            lg, lo = p.forward(np.array([int(rng.integers(0, 4096))], np.int32), n - 1)
        else:
            lg, lo = p.forward(rng.integers(0, 4096, n).astype(np.int32), 0)
        assert bits_equal(lg, lo), (s, maxdiff(lg, lo))
        toks.append(int(np.argmax(lo[-1])))
        pos.append(n)
    for step in range(3):
        log(f"mixed-length multi-session step {step}, kv_type {kv_type}, positions {pos}")
        lg = np.zeros((4, 4096), np.float32)
        got = np.full(4, -1, np.int32)
        rc = eng.dpuf_amd_engine_forward_slots(p.g, 4, M.ptr(slots), M.ptr(np.array(toks, np.int32)),
                                              M.ptr(np.array(pos, np.int32)), M.ptr(lg), M.ptr(got))
        assert rc == 0, (rc, eng.dpuf_amd_last_error())
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
