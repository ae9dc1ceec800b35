"""Why the engine reproduces the reference's fp32 operation order bit for bit
instead of aiming at the workloads' stated 1e-3 relative / 1e-4 absolute
tolerance: on the Qwen3-0.6B shape (28 layers, hidden 1024, vocab 151936),
the oracle with only its RMSNorm sum of squares reordered (a pairwise tree,
as accurate as the reference's eight fma lanes) already moves the first
decode step's logits past that tolerance, and greedy ids diverge within 32
tokens: the int8 re-quantisation after every norm turns a last-bit change
into whole quantisation steps, and the top-1 / top-2 logit gaps of
random-init weights are small.  A faster engine with reordered reductions
would therefore fail the 32-token greedy-id requirement."""
import numpy as np
import pytest

from dpuf_amd import model as M


@pytest.mark.timeout(600)
def test_norm_order_moves_logits_and_greedy_ids(orc):
    shape = M.QWEN3_0_6B
    V = shape["vocab_size"]
    m = M.Model.build(shape, max_seq_len=80, seed=1234)
    ids = np.random.default_rng(2024).integers(0, V, 32).astype(np.int32)

    def run(tree):
        orc.orc_set_norm_order(tree)
        e = orc.orc_engine_create(*m.create_args())
        lo = np.zeros(V, np.float32)
        assert orc.orc_engine_forward(e, 32, M.ptr(ids), 0, None, 1, M.ptr(lo)) == 0
        toks, first = [], lo.copy()
        for s in range(32):
            tok = int(np.argmax(lo))
            toks.append(tok)
            assert orc.orc_engine_forward(e, 1, M.ptr(np.array([tok], np.int32)), 32 + s, None, 1, M.ptr(lo)) == 0
        orc.orc_engine_destroy(e)
        return toks, first

    try:
        a, la = run(0)
        b, lb = run(1)
    finally:
        orc.orc_set_norm_order(0)
    rel = float(np.max(np.abs(la - lb)) / np.max(np.abs(la)))
    div = next((i for i in range(32) if a[i] != b[i]), None)
    print(f"step-0 max |dlogit| / max |logit| = {rel:.4f}; greedy ids equal {sum(x == y for x, y in zip(a, b))}"
          f" of 32, first divergence at step {div}")
    assert rel > 1e-3  # beyond the stated relative tolerance already at the first step
    assert div is not None and div < 32  # greedy ids diverge within tg32
