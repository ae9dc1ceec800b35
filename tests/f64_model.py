"""A float64 Qwen3 decoder written from the mathematics, for pinning the
oracle's engine composition (oracle/oracle.c orc_engine_forward).

Test infrastructure only.  It shares no code with the oracle: every matrix is
read back row by row through the embedding path (row r of a Mode 12 matrix is
sign * FWHT64((u - 8) * ws), of a Mode 13 / 14 matrix sign * FWHT64(m + u d):
the dense weight the packed bytes stand for), and
the block is the textbook Qwen3 decoder layer:

    h_0 = E[ids] (or the caller's embedding rows)
    per layer:  x = RMSNorm(h) * w_attn
                q, k, v = Wq x, Wk x, Wv x
                per head: RMSNorm over head_dim (QK-norm), NeoX RoPE at the position
                causal GQA: query head j reads kv head j // (n_q / n_kv)
                h = h + Wo attn
                x = RMSNorm(h) * w_ffn
                s = silu(Wg x) * (Wu x), |s| < dead zone -> 0
                h = h + Wd s   (rows past the kept down tiles are zero)
    logits = Wlm (RMSNorm(h) * w_out); Zone-A early exit fills -1e9 past the zone

Activations are not quantised here, so the oracle differs from this model by
its int8 activation noise only.  With kv_q8 the cache holds K and V as the
int8 KV cache represents them: each 32-value block rounded to multiples of
amax / 127.  `mut` switches on one deliberate mistake at a
time; the pinning test checks that each one is caught.
"""
import ctypes as C

import numpy as np

from dpuf_amd import model as M


def dense(orc, d):
    """Dense [rows, cols] float64 weight of a Mode 12, 13 or 14 descriptor."""
    ids = np.arange(d.rows, dtype=np.int32)
    out = np.zeros((d.rows, d.cols), np.float32)
    orc.orc_embed_desc(C.byref(d), d.rows, M.ptr(ids), M.ptr(out))
    return out.astype(np.float64)


def _vec(p, n):
    return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_float)), (n,)).astype(np.float64)


class F64Model:
    def __init__(self, orc, model):
        c = model.cfg.contents
        self.H, self.I, self.L = c.hidden_size, c.intermediate_size, c.num_layers
        self.nq, self.nkv, self.hd = c.num_q_heads, c.num_kv_heads, c.head_dim
        self.V, self.eps, self.theta = c.vocab_size, float(c.rms_eps), float(c.rope_theta)
        self.has_qk_norm = bool(c.has_qk_norm)
        self.E = dense(orc, model.tok.contents)
        self.Wlm = dense(orc, model.lm.contents)
        self.out_norm = _vec(model.out_norm, self.H)
        self.layers = []
        for l in range(self.L):
            lw = model.layers[l]
            W = {n: dense(orc, getattr(lw, "w_" + n)) for n in ("q", "k", "v", "o", "gate", "up", "down")}
            W["attn_norm"] = _vec(lw.attn_norm, self.H)
            W["ffn_norm"] = _vec(lw.ffn_norm, self.H)
            W["q_norm"] = _vec(lw.attn_q_norm, self.hd) if lw.attn_q_norm else None
            W["k_norm"] = _vec(lw.attn_k_norm, self.hd) if lw.attn_k_norm else None
            W["down_tiles"] = lw.w_down.n_tiles
            self.layers.append(W)
        self.reset()

    def q8(self, x, mut=()):
        """Per-32-block int8 round trip of the last axis: q = round(x * 127 /
        amax) clamped to [-127, 127], value q * amax / 127 (amax <= 1e-12: 0)."""
        shp = x.shape
        b = x.reshape(-1, 32)
        amax = np.max(np.abs(b), axis=1, keepdims=True)
        inv = np.where(amax > 1e-12, 127.0 / np.where(amax > 0, amax, 1.0), 0.0)
        q = np.clip(np.round(b * inv), -127, 127)
        sc = amax / 127.0
        if "q8_scale_shift" in mut:  # the scale of the neighbouring block
            sc = np.roll(sc.reshape(-1, self.hd // 32), 1, axis=1).reshape(-1, 1)
        return (q * sc).reshape(shp)

    def reset(self):
        self.kc = np.zeros((self.L, self.nkv, 0, self.hd))
        self.vc = np.zeros((self.L, self.nkv, 0, self.hd))

    def set_kv(self, layer, kvh, pos0, k, v, kv_q8=False):
        if kv_q8:
            k, v = self.q8(k), self.q8(v)
        n = k.shape[0]
        need = pos0 + n
        if self.kc.shape[2] < need:
            pad = need - self.kc.shape[2]
            z = np.zeros((self.L, self.nkv, pad, self.hd))
            self.kc = np.concatenate([self.kc, z], axis=2)
            self.vc = np.concatenate([self.vc, z.copy()], axis=2)
        self.kc[layer, kvh, pos0:need] = k
        self.vc[layer, kvh, pos0:need] = v

    def _norm(self, x, w, mut):
        if "norm_no_eps" in mut:
            return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True)) * w
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps) * w

    def _rope(self, x, pos, mut):
        """NeoX rotation of the last axis (pairs j, j + hd/2) by pos * theta^(-2j/hd)."""
        half = self.hd // 2
        j = np.arange(half)
        ang = pos * (1.0 / self.theta ** (2.0 * j / self.hd))
        c, s = np.cos(ang), np.sin(ang)
        if "rope_interleaved" in mut:
            x1, x2 = x[..., 0::2], x[..., 1::2]
            out = np.empty_like(x)
            out[..., 0::2] = x1 * c - x2 * s
            out[..., 1::2] = x2 * c + x1 * s
            return out
        x1, x2 = x[..., :half], x[..., half:]
        if "rope_sign" in mut:
            s = -s
        return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)

    def forward(self, ids, pos0, embeds=None, keep_tiles=0, deadzone=0.005, early=None, mut=(), capture=None,
                kv_q8=False):
        """Returns logits [M, V] of every row; capture (a list) receives the
        residual stream after each layer, [M, H] per layer."""
        mut = set(mut)
        M_ = len(ids) if ids is not None else embeds.shape[0]
        if ids is None:
            h = embeds.astype(np.float64).copy()
        else:
            h = np.stack([embeds[m] if (embeds is not None and ids[m] < 0) else self.E[ids[m]]
                          for m in range(M_)]).astype(np.float64)
        nq, nkv, hd, G = self.nq, self.nkv, self.hd, self.nq // self.nkv
        end = pos0 + M_
        if self.kc.shape[2] < end:
            pad = end - self.kc.shape[2]
            z = np.zeros((self.L, nkv, pad, hd))
            self.kc = np.concatenate([self.kc, z], axis=2)
            self.vc = np.concatenate([self.vc, z.copy()], axis=2)
        for l, W in enumerate(self.layers):
            x = self._norm(h, W["attn_norm"], mut)
            q = (x @ W["q"].T).reshape(M_, nq, hd)
            k = (x @ W["k"].T).reshape(M_, nkv, hd)
            v = (x @ W["v"].T).reshape(M_, nkv, hd)
            if self.has_qk_norm and "no_qk_norm" not in mut:
                q = self._norm(q, W["q_norm"], mut)
                k = self._norm(k, W["k_norm"], mut)
            pos = np.arange(pos0, end)[:, None, None]
            q = self._rope(q, pos, mut)
            k = self._rope(k, pos, mut)
            if kv_q8:
                k, v = self.q8(k, mut), self.q8(v, mut)
            self.kc[l, :, pos0:end] = k.transpose(1, 0, 2)
            self.vc[l, :, pos0:end] = v.transpose(1, 0, 2)
            ao = np.zeros((M_, nq, hd))
            for m in range(M_):
                n = pos0 + m + (0 if "causal_off_by_one" in mut else 1)
                n = max(n, 1)
                for j in range(nq):
                    kvh = (j % nkv) if "gqa_modulo" in mut else j // G
                    s = self.kc[l, kvh, :n] @ q[m, j] / np.sqrt(hd)
                    p = np.exp(s - s.max())
                    p /= p.sum()
                    ao[m, j] = p @ self.vc[l, kvh, :n]
            o = ao.reshape(M_, nq * hd) @ W["o"].T
            if "no_attn_residual" in mut:
                h = o
            else:
                h = h + o
            x = self._norm(h, W["ffn_norm"], mut)
            g, u = x @ W["gate"].T, x @ W["up"].T
            if "swiglu_swapped" in mut:
                g, u = u, g
            s = g / (1.0 + np.exp(-np.clip(g, -40, 40))) * u
            if deadzone > 0 and "no_deadzone" not in mut:
                s = np.where(np.abs(s) < deadzone, 0.0, s)
            dn = s @ W["down"].T
            nt = W["down_tiles"]
            if 0 < keep_tiles < nt and "prune_unzeroed" not in mut:
                dn[:, keep_tiles * 16:] = 0.0
            h = h + dn
            if capture is not None:
                capture.append(h.copy())
        x = self._norm(h, self.out_norm, mut)
        logits = x @ self.Wlm.T
        if early is not None:
            zone_tiles, margin = early
            nz = min(zone_tiles * 16, self.V)
            top = np.sort(logits[-1, :nz])[::-1]
            if margin > 0 and top[0] - top[1] >= margin:
                logits[-1, nz:] = -1e30 if "fill_wrong" in mut else -1e9
        return logits
