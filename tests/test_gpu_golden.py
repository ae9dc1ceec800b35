"""GPU results against the committed golden fixtures (tests/golden/*.npz):
the standalone Mode 12 entry points and the engine's greedy decode, bit for
bit, through the C ABI."""
import os

import numpy as np
import pytest

from dpuf_amd import model as M

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_gemv_fixture(eng):
    g = load("gemv_40x256.npz")
    tiles, offs, sign = g["tiles"].copy(), g["offs"].copy(), g["sign"].copy()
    rows, cols, nt = int(g["rows"]), int(g["cols"]), int(g["n_tiles"])
    x = g["x"].copy()
    print("golden gemv 40x256", flush=True)
    for Mm, key in ((3, "out_m3"), (1, "out_m1")):
        out = np.full((Mm, rows), np.nan, np.float32)
        eng.dpuf_matmul_qr_hadamard4_packed_f32(Mm, rows, cols, nt, M.ptr(x[:Mm]), M.ptr(tiles), M.ptr(offs),
                                                M.ptr(sign), M.ptr(out))
        assert np.array_equal(bits(out), bits(g[key][:Mm]))
    f = np.zeros(cols, np.float32)
    eng.dpuf_fwht64_sign_f32(cols, M.ptr(x[0]), M.ptr(sign), M.ptr(f))
    assert np.array_equal(bits(f), bits(g["fwht0"]))
    emb = np.zeros((4, cols), np.float32)
    ids = g["embed_ids"].copy()
    eng.dpuf_embed_qr_hadamard4_packed_f32(4, cols, M.ptr(ids), M.ptr(tiles), M.ptr(offs), M.ptr(sign), M.ptr(emb))
    assert np.array_equal(bits(emb), bits(g["embed"]))


def test_engine_fixture(eng):
    g = load("engine_tiny.npz")
    keys = ("hidden_size", "intermediate_size", "num_layers", "num_q_heads", "num_kv_heads", "head_dim",
            "vocab_size", "tie_word_embeddings")
    shape = {k: int(v) for k, v in zip(keys, g["shape"])}
    m = M.Model.build(shape, max_seq_len=int(g["max_seq"]), seed=int(g["seed"]))
    h = eng.dpuf_engine_create(*m.create_args())
    assert h, eng.dpuf_amd_last_error()
    V = shape["vocab_size"]
    prompt = g["prompt"].copy()
    lg = np.zeros((8, V), np.float32)
    print("golden engine prefill 8", flush=True)
    assert eng.dpuf_engine_forward_batch(h, 8, M.ptr(prompt), 0, 0, M.ptr(lg)) == 0
    assert np.array_equal(bits(lg), bits(g["prefill_logits"]))
    lo = np.zeros(V, np.float32)
    got = []
    tok = int(np.argmax(lg[-1]))
    for step in range(len(g["greedy_ids"])):
        got.append(tok)
        assert eng.dpuf_engine_forward_token(h, tok, 8 + step, M.ptr(lo)) == 0
        assert np.array_equal(bits(lo), bits(g["step_logits"][step])), step
        tok = int(np.argmax(lo))
    assert got == list(g["greedy_ids"])
    eng.dpuf_engine_destroy(h)
