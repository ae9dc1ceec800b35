"""The oracle and the packer reproduce the committed golden fixtures
(tests/golden/*.npz, written by tests/golden/make_golden.py) bit for bit."""
import os

import numpy as np

from dpuf_amd import model as M

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_packer_reproduces_fixture_tiles():
    g = load("gemv_40x256.npz")
    W = M.random_normal(40 * 256, 0.02, 31, "golden-w").reshape(40, 256)
    sb = M.sign_bits(256, 31, "golden-s")
    blob, d = M.pack_matrix(W, sb)
    tiles, offs, s = M.desc_arrays(d)
    assert np.array_equal(tiles, g["tiles"]) and np.array_equal(offs, g["offs"]) and np.array_equal(s, g["sign"])


def test_oracle_reproduces_gemv_fixture(orc):
    g = load("gemv_40x256.npz")
    tiles, offs, sign = g["tiles"].copy(), g["offs"].copy(), g["sign"].copy()
    rows, cols, nt = int(g["rows"]), int(g["cols"]), int(g["n_tiles"])
    x = g["x"].copy()
    out = np.zeros((3, rows), np.float32)
    orc.orc_matmul_f32(3, rows, cols, nt, M.ptr(x), M.ptr(tiles), M.ptr(offs), M.ptr(sign), M.ptr(out))
    assert np.array_equal(bits(out), bits(g["out_m3"]))
    assert np.array_equal(bits(g["out_m1"]), bits(g["out_m3"]))  # M = 1 and slab paths agree
    q = np.zeros(cols, np.int8)
    s = np.zeros(cols // 32, np.float32)
    m = np.zeros(cols // 32, np.int32)
    orc.orc_prep_row(cols, M.ptr(x[0]), M.ptr(sign), M.ptr(q), M.ptr(s), M.ptr(m))
    assert np.array_equal(q, g["q0"]) and np.array_equal(bits(s), bits(g["s0"])) and np.array_equal(m, g["m0"])
    emb = np.zeros((4, cols), np.float32)
    ids = g["embed_ids"].copy()
    orc.orc_embed(4, cols, M.ptr(ids), M.ptr(tiles), M.ptr(offs), M.ptr(sign), M.ptr(emb))
    assert np.array_equal(bits(emb), bits(g["embed"]))


def tiny_shape(g):
    keys = ("hidden_size", "intermediate_size", "num_layers", "num_q_heads", "num_kv_heads", "head_dim",
            "vocab_size", "tie_word_embeddings")
    return {k: int(v) for k, v in zip(keys, g["shape"])}


def test_oracle_reproduces_engine_fixture(orc, tools):
    g = load("engine_tiny.npz")
    m = M.Model.build(tiny_shape(g), max_seq_len=int(g["max_seq"]), seed=int(g["seed"]))
    crc = 0
    for l in range(int(g["shape"][2])):
        t, _, _ = M.desc_arrays(m.layers[l].w_down)
        crc ^= tools.dpuf_crc32_bytes(M.ptr(np.ascontiguousarray(t)), t.size)
    assert crc == int(g["down_tiles_crc"])
    h = orc.orc_engine_create(*m.create_args())
    V = int(g["shape"][6])
    prompt = g["prompt"].copy()
    lg = np.zeros((8, V), np.float32)
    assert orc.orc_engine_forward(h, 8, M.ptr(prompt), 0, None, 0, M.ptr(lg)) == 0
    assert np.array_equal(bits(lg), bits(g["prefill_logits"]))
    ids = g["greedy_ids"]
    lo = np.zeros(V, np.float32)
    one = np.zeros(1, np.int32)
    for step in range(len(ids)):
        one[0] = ids[step]
        assert orc.orc_engine_forward(h, 1, M.ptr(one), 8 + step, None, 1, M.ptr(lo)) == 0
        assert np.array_equal(bits(lo), bits(g["step_logits"][step]))
    orc.orc_engine_destroy(h)
