// attn_common.h -- device helpers and launch constants shared by the attention
// translation units (attn.hip, attn_wide.hip).
#ifndef DPUF_ATTN_COMMON_H
#define DPUF_ATTN_COMMON_H

#include "dev_common.h"
#include "dev_exp.h"

// ---------------------------------------------------------------------------
// QK-norm + NeoX RoPE + KV-cache store (reference dpuf_engine.c:1791-1817,
// 1841-1879).  grid: (M, n_q + n_kv); block: hd threads.
// ---------------------------------------------------------------------------
// The same per (token, head) with one wave each, four per workgroup, for
// HD = 64, 128, 256: lane l holds elements l + 64e (e < HD / 64), so a RoPE
// pair (i, i + HD/2) sits in one lane for HD >= 128 and in lanes l, l ^ 32
// for HD = 64; the norm's 8 accumulator chains (lane j: elements j, j + 8,
// ... in order) gather their elements by shuffles, the hsum tree follows.
// Int8 KV cache store of one value per lane (quantize_vec_q8_blk32,
// dpuf_engine.c:754-781): a wave's lanes 0-31 and 32-63 each hold one
// 32-block (elements 64e .. 64e+31 and 64e+32 .. 64e+63); amax over the half
// wave, q = RNE(x * (127 / amax)) saturated to [-127, 127] (a value the
// conversion cannot represent gives -127), scale amax / 127 stored by the
// half's first lane.  amax <= 1e-12 gives q = 0.
DEV void q8_store_lane(float val, int lane, int e, int8_t* row, float* srow) {
    float a = fabsf(val);
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
    const float inv = a > 1e-12f ? 127.0f / a : 0.0f;
    const float x = val * inv;
    int qv;
    if (!(x > -2147483648.0f && x < 2147483648.0f)) qv = -127;
    else qv = (int)rintf(x);
    qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
    row[lane + 64 * e] = (int8_t)qv;
    if ((lane & 31) == 0) srow[2 * e + (lane >> 5)] = a / 127.0f;
}

// QK-norm (reference rms_norm_f32 over one head, dpuf_engine.c:225-241) and
// NeoX RoPE of one head by one wave, element i = lane + 64 e in x[e]: the
// inputs come from qk_head_load (every load first, one memory round trip).
template <int HD>
struct QkHead {
    float x[HD / 64], wn[HD / 64], cs[HD / 64], sn[HD / 64];
};

template <int HD>
DEV void qk_head_load(const float* vec, const float* nw, const float* cos_tab, const float* sin_tab, int pos, int lane,
                      QkHead<HD>& h) {
    constexpr int E = HD / 64, half = HD / 2;
#pragma unroll
    for (int e = 0; e < E; e++) {
        const int i = lane + 64 * e, j = i < half ? i : i - half;
        h.x[e] = vec[i];
        h.wn[e] = nw ? nw[i] : 1.0f;
        h.cs[e] = cos_tab[(size_t)pos * half + j];
        h.sn[e] = sin_tab[(size_t)pos * half + j];
    }
}

template <int HD>
DEV void qk_head_rope(QkHead<HD>& h, bool norm, float eps, int lane, float (&o)[HD / 64]) {
    constexpr int E = HD / 64, half = HD / 2;
    if (norm) {
        // chain j = lane (< 8): elements j + 8i, i = 0 .. HD/8 - 1, in order
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < HD / 8; i++) {
            // element (lane & 7) + 8i: register i / 8 of lane (lane & 7) + 8 (i % 8)
            const float xv = __shfl(h.x[i / 8], (lane & 7) + 8 * (i % 8), 64);
            a = fmaf(xv, xv, a);
        }
        float pt[8];
#pragma unroll
        for (int j = 0; j < 8; j++) pt[j] = __shfl(a, j, 64);
        const float inv = 1.0f / sqrtf(hsum8(pt) / (float)HD + eps);
#pragma unroll
        for (int e = 0; e < E; e++) h.x[e] = (h.x[e] * inv) * h.wn[e];
    }
#pragma unroll
    for (int e = 0; e < E; e++) {
        const int i = lane + 64 * e;
        float partner;
        if (E == 1) partner = __shfl_xor(h.x[0], 32, 64);  // element i ^ 32 = i +- half
        else partner = h.x[i < half ? e + E / 2 : e - E / 2];
        if (i < half) o[e] = fmaf(h.x[e], h.cs[e], -(partner * h.sn[e]));
        else o[e] = fmaf(h.x[e], h.cs[e], partner * h.sn[e]);
    }
}


DEV float score_hadd(const float* q, const float* kp, int hd) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < hd; i += 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = fmaf(q[i + j], kp[i + j], a[j]);
    }
    return hsum8_hadd(a);
}
DEV float score_hsum(const float* q, const float* kp, int hd) {
    float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < hd; i += 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) a[j] = fmaf(q[i + j], kp[i + j], a[j]);
    }
    return hsum8(a);
}
// dot_f32_avx2 (dpuf_engine.c:325-339) for the single-head tail.
DEV float score_dot2(const float* q, const float* kp, int hd) {
    float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; i + 15 < hd; i += 16) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            a0[j] = fmaf(q[i + j], kp[i + j], a0[j]);
            a1[j] = fmaf(q[i + 8 + j], kp[i + 8 + j], a1[j]);
        }
    }
    for (; i + 7 < hd; i += 8) {
#pragma unroll
        for (int j = 0; j < 8; j++) a0[j] = fmaf(q[i + j], kp[i + j], a0[j]);
    }
    float cc[8];
#pragma unroll
    for (int j = 0; j < 8; j++) cc[j] = a0[j] + a1[j];
    return hsum8(cc);
}


// ---------------------------------------------------------------------------
// Split attention for prefill and long-context decode: the same arithmetic as
// gqa_attn_head_pair_f32 (dpuf_engine.c:341-577) spread over the GPU.
//
// k_attn_sc: scores.  Workgroup (kv head, tile of qt queries, 64 keys): the
// key chunk and the tile's q rows (qt x G heads, <= 32 rows) are staged in
// LDS; thread (rp, kq) forms rows 2rp, 2rp + 1 against keys kq + 16b, b < 4, as
// the reference's 8-lane accumulators (a[j] = fma chain over i of
// q[8i + j] * k[8i + j]), then applies the reference's horizontal sum for
// that (query, key): the hadd tree for keys below kv_len & ~3, eng_hsum256
// above it (dot_f32_avx2's two-accumulator form for a single trailing head),
// times the scale.  Writes S[m][head][t] for t < kv_len(m) = pos0 + m + 1.

// keys per workgroup of the scores kernels
#define AS_KC 64  // keys per scores workgroup

// ROPE: q, k and v are the projections' raw rows; the workgroup applies the
// QK-norm and RoPE to its group's q rows itself (as k_qk_rope_kv_w does, by
// qk_head_rope), and the workgroup whose chunk holds the token's position
// does the same to its K row, stores K and V to the cache at that position
// and uses the new K row in its scores (so no launch before this one).
struct ScRope {
    const float* k;  // raw K and V of the token [n_kv][HD]
    const float* v;
    const float* qn;  // QK-norm weights (NULL: no norm)
    const float* kn;
    float eps;
    const float* cos_tab;
    const float* sin_tab;
    float* kc;  // the cache rows written at the position
    float* vc;
};

// ---------------------------------------------------------------------------
// k_attn_pv: softmax and P.V.  Workgroup (kv head, tile of qt queries, dim
// chunk of HD / dc): the tile's score rows (R = qt x G, each kv_len(m) long)
// are read into LDS and turned into probabilities as the reference does
// (max; exp polynomial on the 8-aligned part, expf on the tail; the 8-lane
// sum chains + eng_hsum256 + the tail added in order; 1 / (sum + 1e-12);
// multiply, in place), then thread (r, d) runs the row's P.V chain for dim d over the
// keys in order (nested pairs for a single trailing head, as the reference's
// single-head path), V staged in LDS in chunks of vk keys.  Every dim chunk
// recomputes its rows' softmax (cheap next to P.V).
// ---------------------------------------------------------------------------
// Sequential chain a = a + x[0] + x[step] + x[2 step] ... over n LDS values,
// read in batches of 16 with the next batch in flight.
DEV float lds_sum_chain(const float* x, int step, int n) {
    float a = 0.0f;
    int k = 0;
    if (n >= 32) {
        float cur[16], nxt[16];
#pragma unroll
        for (int i = 0; i < 16; i++) cur[i] = x[i * step];
        for (k = 16; k + 16 <= n; k += 16) {
#pragma unroll
            for (int i = 0; i < 16; i++) nxt[i] = x[(k + i) * step];
#pragma unroll
            for (int i = 0; i < 16; i++) a = a + cur[i];
#pragma unroll
            for (int i = 0; i < 16; i++) cur[i] = nxt[i];
        }
#pragma unroll
        for (int i = 0; i < 16; i++) a = a + cur[i];
    }
    for (; k < n; k++) a = a + x[k * step];
    return a;
}

// P.V chain of one (row, dim) over n keys of a chunk, in key order, with the
// normalised probabilities p[t]: a = fma(p[t], v[t], a), or the nested pairs
// a = fma(p[t], v[t], fma(p[t+1], v[t+1], a)) of the reference's
// single-head path.  p and v are
// 16-byte aligned LDS rows (v: this dim's values for consecutive keys); keys
// go in batches of 16 from two alternating register sets, so one batch's
// reads are in flight while the other's FMAs run.
DEV void pv_load16(const float* p, const float* v, int t, float4 (&pb)[4], float4 (&vb)[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        pb[i] = *(const float4*)(p + t + 4 * i);
        vb[i] = *(const float4*)(v + t + 4 * i);
    }
}

template <bool NESTED>
DEV float pv_fma16(const float4 (&pb)[4], const float4 (&vb)[4], float a) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float p0 = pb[i].x, p1 = pb[i].y, p2 = pb[i].z, p3 = pb[i].w;
        if (NESTED) {
            a = fmaf(p0, vb[i].x, fmaf(p1, vb[i].y, a));
            a = fmaf(p2, vb[i].z, fmaf(p3, vb[i].w, a));
        } else {
            a = fmaf(p0, vb[i].x, a);
            a = fmaf(p1, vb[i].y, a);
            a = fmaf(p2, vb[i].z, a);
            a = fmaf(p3, vb[i].w, a);
        }
    }
    return a;
}

template <bool NESTED>
DEV float pv_chain(const float* p, const float* v, int n, float a) {
    const int n16 = n & ~15;
    int t = 0;
    if (n16 > 0) {
        float4 pa[4], va[4], pb[4], vb[4];
        pv_load16(p, v, 0, pa, va);
        for (t = 0; t + 32 <= n16; t += 32) {
            pv_load16(p, v, t + 16, pb, vb);
            __builtin_amdgcn_sched_barrier(0);  // keep the next batch's reads ahead of these FMAs
            a = pv_fma16<NESTED>(pa, va, a);
            pv_load16(p, v, t + 32 < n16 ? t + 32 : t, pa, va);  // the last reload is unused
            __builtin_amdgcn_sched_barrier(0);
            a = pv_fma16<NESTED>(pb, vb, a);
        }
        if (t < n16) {
            a = pv_fma16<NESTED>(pa, va, a);
            t += 16;
        }
    }
    if (NESTED) {
        for (; t + 1 < n; t += 2) a = fmaf(p[t], v[t], fmaf(p[t + 1], v[t + 1], a));
        if (t < n) a = fmaf(p[t], v[t], a);
    } else {
        for (; t < n; t++) a = fmaf(p[t], v[t], a);
    }
    return a;
}

// With Q8 (the int8 KV cache) V comes from vq / vsc instead of vc: the dim
// chunk lies inside one 32-column block (dw <= 32), its int8 values are
// widened to floats in LDS (exact), and per chunk W[r][t] = p[r][t] * vs[t]
// (the reference's p * v_scale, dpuf_engine.c:726-747) takes p's place in the
// chains.

// The one-token long-context kernels (attn_wide.hip): fp32 cache scores
// (with the QK-norm, RoPE and KV store when rope is set), softmax once per row
// and the wide P.V; -1 (nothing launched) when the shape does not take them.
// wm (or NULL): the weight groups that warm-up workgroups of the P.V launch
// read into the caches on the CUs its chain workgroups leave idle.
int32_t attn_wide_f32(void* s, int32_t lmax, const float* q, const float* kc, const float* vc, float* out,
                      float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                      float scale, const ScRope* rope, const DpufWarm* wm);
// The int8 cache's softmax once per row + wide P.V after its scores kernel;
// -1 (nothing launched) when the shape does not take them.  wm (or NULL):
// weights that warm-up workgroups of the P.V launch read into the caches.
int32_t attn_wide_q8(void* s, int32_t lmax, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd,
                     int32_t max_seq, float* scores, float* out, DpufKvQ8 c8, const DpufWarm* wm);

// Warm-up workgroup i (of wm.n_wg; grid position L, so XCD L % 8): the
// units of its XCD are (job j, round lg, the k-th workgroup of job j on that
// XCD), job by job; it takes a share of at most WARM_MAXU of them, puts their
// group addresses and sizes in LDS, and reads the groups with 16-byte loads,
// WARM_DEPTH in flight per lane.  Called by every thread of the workgroup.
#define WARM_MAXU 48
#define WARM_DEPTH 32  // loads in flight per lane (16 and 64 measured slower)
DEV void warm_read(const DpufWarm& wm, int i, int L, int tid, int nthr) {
    __shared__ const uint8_t* gtab[WARM_MAXU];
    __shared__ int gqt[WARM_MAXU];
    const int x = L & 7, r = i >> 3, per_x = wm.n_wg >> 3;
    if (per_x <= 0 || wm.n_jobs <= 0) return;
    int U = 0;
    for (int j = 0; j < wm.n_jobs; j++) {
        const DpufWarmJob& J = wm.j[j];
        const int c = (x - J.wb) & 7;
        if ((J.group_bytes >> 4) < nthr) return;  // one wrap per step below
        U += (J.nwg > c ? (J.nwg - c + 7) >> 3 : 0) * J.nr;
    }
    if (U <= 0) return;
    const int tp = (U + per_x - 1) / per_x, u0 = r * tp;
    int nu = U - u0 < tp ? U - u0 : tp;
    if (nu > WARM_MAXU) nu = WARM_MAXU;
    if (nu <= 0) return;
    if (tid < nu) {
        int u = u0 + tid;
        const uint8_t* gp = nullptr;
        int gq = 0;
        for (int j = 0; j < wm.n_jobs; j++) {
            const DpufWarmJob& J = wm.j[j];
            const int c = (x - J.wb) & 7, cnt = J.nwg > c ? (J.nwg - c + 7) >> 3 : 0;
            if (u < cnt * J.nr) {
                const int lg = J.r0 + u / cnt, k = u - (u / cnt) * cnt;
                const int g = c + 8 * k + lg * J.nwg;
                if (g < J.n_groups) gp = J.p + (size_t)g * J.group_bytes;
                gq = J.group_bytes >> 4;
                break;
            }
            u -= cnt * J.nr;
        }
        gtab[tid] = gp;
        gqt[tid] = gq > 0 ? gq : nthr;
    }
    __syncthreads();
    int t = 0, o = tid;
    uint32_t acc = 0;
    while (t < nu) {
        uint4 v[WARM_DEPTH];
#pragma unroll
        for (int k = 0; k < WARM_DEPTH; k++) {
            v[k] = make_uint4(0u, 0u, 0u, 0u);
            if (t < nu) {
                const uint8_t* gp = gtab[t];
                const int gq = gqt[t];
                if (gp) v[k] = ((const uint4*)gp)[o];
                o += nthr;  // nthr <= gq: at most one wrap
                const bool wr = o >= gq;
                o = wr ? o - gq : o;
                t += wr ? 1 : 0;
            }
        }
#pragma unroll
        for (int k = 0; k < WARM_DEPTH; k++) acc ^= v[k].x ^ v[k].w;
    }
    if (acc == 0x9E3779B9u) *wm.sink = (int32_t)acc;
}

#endif
