"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

The reference holds no fixture for the Mode 12 path, so these vectors are
outputs of the oracle (oracle/oracle.c, itself pinned by tests/test_cpu_oracle.py)
on seeded inputs.  They freeze the expected results so that GPU runs can be
checked against stored data as well as against a live oracle run, and so
that a change to the oracle or to the packer shows up as a fixture diff.

Run from the repository root:  python tests/golden/make_golden.py
"""
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from dpuf_amd import model as M  # noqa: E402
from oracle import oracle as O  # noqa: E402

TINY = dict(hidden_size=256, intermediate_size=512, num_layers=3, num_q_heads=4, num_kv_heads=2, head_dim=64,
            vocab_size=4096, tie_word_embeddings=1)
TINY_SEED, TINY_SEQ = 77, 64


def gemv_fixture(orc):
    rows, cols = 40, 256
    W = M.random_normal(rows * cols, 0.02, 31, "golden-w").reshape(rows, cols)
    sb = M.sign_bits(cols, 31, "golden-s")
    blob, d = M.pack_matrix(W, sb)
    tiles, offs, _ = M.desc_arrays(d)
    rng = np.random.default_rng(2024)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    x[1, 64:96] = 1e-6  # a zero-scale block
    out3 = np.zeros((3, rows), np.float32)
    orc.orc_matmul_f32(3, rows, cols, d.n_tiles, M.ptr(x), d.tensor_base, d.tile_offsets, d.sign_bits, M.ptr(out3))
    out1 = np.zeros((3, rows), np.float32)
    for i in range(3):
        orc.orc_matmul_f32(1, rows, cols, d.n_tiles, M.ptr(np.ascontiguousarray(x[i])), d.tensor_base,
                           d.tile_offsets, d.sign_bits, M.ptr(out1[i]))
    f = np.zeros(cols, np.float32)
    orc.orc_fwht64_sign(cols, M.ptr(x[0]), d.sign_bits, M.ptr(f))
    q = np.zeros(cols, np.int8)
    s = np.zeros(cols // 32, np.float32)
    m = np.zeros(cols // 32, np.int32)
    orc.orc_prep_row(cols, M.ptr(x[0]), d.sign_bits, M.ptr(q), M.ptr(s), M.ptr(m))
    ids = np.array([0, 5, 16, 39], np.int32)
    emb = np.zeros((4, cols), np.float32)
    orc.orc_embed(4, cols, M.ptr(ids), d.tensor_base, d.tile_offsets, d.sign_bits, M.ptr(emb))
    np.savez_compressed(os.path.join(HERE, "gemv_40x256.npz"), rows=rows, cols=cols, n_tiles=d.n_tiles,
                        tiles=tiles.copy(), offs=offs.copy(), sign=sb, x=x, out_m1=out1, out_m3=out3, fwht0=f,
                        q0=q, s0=s, m0=m, embed_ids=ids, embed=emb)


def engine_fixture(orc):
    m = M.Model.build(TINY, max_seq_len=TINY_SEQ, seed=TINY_SEED)
    h = orc.orc_engine_create(*m.create_args())
    V = TINY["vocab_size"]
    prompt = np.random.default_rng(5).integers(0, V, 8).astype(np.int32)
    lg = np.zeros((8, V), np.float32)
    assert orc.orc_engine_forward(h, 8, M.ptr(prompt), 0, None, 0, M.ptr(lg)) == 0
    first = lg.copy()
    ids = []
    tok = int(np.argmax(lg[-1]))
    step_logits = []
    one = np.zeros(1, np.int32)
    lo = np.zeros(V, np.float32)
    for step in range(8):
        ids.append(tok)
        one[0] = tok
        assert orc.orc_engine_forward(h, 1, M.ptr(one), 8 + step, None, 1, M.ptr(lo)) == 0
        step_logits.append(lo.copy())
        tok = orc.orc_argmax(M.ptr(lo), V)
    orc.orc_engine_destroy(h)
    crc = 0
    lib = M.abi.load_tools()
    for l in range(TINY["num_layers"]):
        t, o, _ = M.desc_arrays(m.layers[l].w_down)
        crc ^= lib.dpuf_crc32_bytes(M.ptr(np.ascontiguousarray(t)), t.size)
    np.savez_compressed(os.path.join(HERE, "engine_tiny.npz"), seed=TINY_SEED, max_seq=TINY_SEQ, prompt=prompt,
                        prefill_logits=first, greedy_ids=np.array(ids, np.int32),
                        step_logits=np.stack(step_logits), down_tiles_crc=np.uint32(crc),
                        shape=np.array([TINY[k] for k in ("hidden_size", "intermediate_size", "num_layers",
                                                          "num_q_heads", "num_kv_heads", "head_dim", "vocab_size",
                                                          "tie_word_embeddings")], np.int32))


if __name__ == "__main__":
    orc = O.load()
    gemv_fixture(orc)
    engine_fixture(orc)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
