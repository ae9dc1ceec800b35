"""Configurations dpuf_engine_create accepts beyond the Qwen3 benchmark
shapes, each bit-exact against the oracle through the C ABI: head_dim 256
(the decode, prefill and long-context attention instances for 256-wide
heads, fp32 and int8 caches) and the Llama-3 RoPE scaling of the rotation
tables (dpuf_engine.c:194-208)."""
import numpy as np
import pytest

from dpuf_amd import abi
from dpuf_amd import model as M
from test_gpu_configs import Pair, bits_equal, greedy, log, maxdiff
from test_gpu_q8kv import Q8Pair

pytestmark = pytest.mark.gpu


def engine_pair(eng, orc, shape, max_seq, seed, **cfg_over):
    m = M.Model.build(shape, max_seq_len=max_seq, seed=seed)
    cfg = abi.DpufModelConfig.from_buffer_copy(m.cfg.contents)
    for k, v in cfg_over.items():
        setattr(cfg, k, v)
    return Q8Pair(eng, orc, m, cfg)


def injected_decode(p, rng, layers, nkv, hd, ctx, steps, what):
    for layer in range(layers):
        for kvh in range(nkv):
            p.set_kv(layer, kvh, 0, rng.standard_normal((ctx, hd), dtype=np.float32),
                     rng.standard_normal((ctx, hd), dtype=np.float32))
    lg, lo = p.forward(np.array([int(rng.integers(0, 4096))], np.int32), ctx)
    assert bits_equal(lg, lo), (what, maxdiff(lg, lo))
    greedy(p, lg, lo, ctx + 1, steps, what)


@pytest.mark.parametrize("kv_type", [0, 1])
def test_head_dim_256(eng, orc, kv_type):
    """head_dim 256 with groups of 2 (Q width 1024 over hidden 512): a
    20-token prefill and 6 greedy steps (fused short-context decode), then a
    second slot with 700 injected keys and 3 steps (the one-token
    long-context kernels), logits bit-identical."""
    shape = dict(hidden_size=512, intermediate_size=1024, num_layers=2, num_q_heads=4, num_kv_heads=2,
                 head_dim=256, vocab_size=4096, tie_word_embeddings=1)
    p = engine_pair(eng, orc, shape, 720, 501, kv_type=kv_type)
    rng = np.random.default_rng(502)
    log(f"head_dim 256, kv_type {kv_type}: pp20 + 6 steps")
    lg, lo = p.forward(rng.integers(0, 4096, 20).astype(np.int32), 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 20, 6, "hd256")
    p.set_slot(1)
    log(f"head_dim 256, kv_type {kv_type}: 700 injected keys + 3 steps")
    injected_decode(p, rng, 2, 2, 256, 700, 3, "hd256 long")
    p.close()


def test_llama3_rope_scaling(eng, orc):
    """use_llama3_rope with Llama-3.1's settings (theta 5e5, factor 8, low 1,
    high 4, original context 8192) at the 8B attention geometry (groups of 4,
    head_dim 128): the engine's rotation tables equal the oracle's, so a
    24-token prefill, 6 greedy steps and 3 steps after 2000 injected keys
    (large angles, long-context kernels) are bit-identical; the same model
    without the scaling gives different logits."""
    shape = dict(hidden_size=256, intermediate_size=512, num_layers=2, num_q_heads=8, num_kv_heads=2,
                 head_dim=128, vocab_size=4096, tie_word_embeddings=1)
    llama3 = dict(use_llama3_rope=1, rope_theta=5e5, rope_factor=8.0, rope_low_freq=1.0, rope_high_freq=4.0,
                  rope_orig_max_pos=8192)
    p = engine_pair(eng, orc, shape, 2016, 511, **llama3)
    rng = np.random.default_rng(512)
    ids = rng.integers(0, 4096, 24).astype(np.int32)
    log("Llama-3 RoPE scaling: pp24 + 6 steps")
    lg, lo = p.forward(ids, 0)
    assert bits_equal(lg, lo), maxdiff(lg, lo)
    greedy(p, lg, lo, 24, 6, "llama3 rope")
    p.set_slot(1)
    log("Llama-3 RoPE scaling: 2000 injected keys + 3 steps")
    injected_decode(p, rng, 2, 2, 128, 2000, 3, "llama3 rope long")
    p.close()
    # the scaling changes the result: the unscaled engine at the same theta differs
    q = engine_pair(eng, orc, shape, 2016, 511, **dict(llama3, use_llama3_rope=0))
    lu, _ = q.forward(ids, 0)
    assert not bits_equal(lu, lg)
    q.close()
