// attn.hip -- attention over the fp32 and int8 KV caches: prefill QK-norm +
// RoPE + KV store, the split scores and softmax / P.V kernels of prefill,
// the int8-cache kernels and the one-pair fallback; launches the one-token
// long-context kernels of attn_wide.hip where they apply.
//
// Numerics contract: every kernel reproduces the fp32 operation order of the
// reference CPU path (dpuf_avx2.c / dpuf_engine.c in dulePan/dpuf) so that
// results are bit-identical, not merely close:
//   * integer parts (nibble x int8 dots) are exact in any order, so they are
//     spread over lanes and reduced with DPP;
//   * every floating-point reduction whose order the reference fixes (the
//     per-row FMA chain over 32-blocks, RMSNorm's 8 FMA lanes + hsum tree,
//     attention's hadd tree, softmax sums, the P.V chain) runs in that order;
//   * build with -ffp-contract=off; fused multiply-adds are explicit fmaf.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "hip_layer.h"
#include "dev_common.h"
#include "hip_internal.h"
#include "attn_common.h"

// ---------------------------------------------------------------------------
// QK-norm + NeoX RoPE + KV-cache store (reference dpuf_engine.c:1791-1817,
// 1841-1879).  grid: (M, n_q + n_kv); block: hd threads.
template <int HD, bool Q8>
__global__ __launch_bounds__(256) void k_qk_rope_kv_w(float* __restrict__ q, float* __restrict__ k,
                                                      const float* __restrict__ v, const float* __restrict__ qn,
                                                      const float* __restrict__ kn, float eps,
                                                      const float* __restrict__ cos_tab,
                                                      const float* __restrict__ sin_tab, float* __restrict__ kc,
                                                      float* __restrict__ vc, const int32_t* __restrict__ pos0p, int M,
                                                      int n_q, int n_kv, int max_seq, DpufKvQ8 c8) {
    constexpr int E = HD / 64;
    const int lane = threadIdx.x & 63;
    const int u = blockIdx.x * 4 + (threadIdx.x >> 6);  // (token, head) unit of this wave
    const int nh = n_q + n_kv;
    if (u >= M * nh) return;  // whole wave
    const int m = u / nh, head = u % nh;
    const int pos = *pos0p + m;
    const bool is_k = head >= n_q;
    const int hh = is_k ? head - n_q : head;
    float* vec = is_k ? (k + ((size_t)m * n_kv + hh) * HD) : (q + ((size_t)m * n_q + hh) * HD);
    const float* nw = is_k ? kn : qn;
    // every load first: one memory round trip for the whole wave
    QkHead<HD> hd_;
    float vv[E];
    qk_head_load<HD>(vec, nw, cos_tab, sin_tab, pos, lane, hd_);
#pragma unroll
    for (int e = 0; e < E; e++) vv[e] = is_k ? v[((size_t)m * n_kv + hh) * HD + lane + 64 * e] : 0.0f;
    float o[E];
    qk_head_rope<HD>(hd_, nw != nullptr, eps, lane, o);
#pragma unroll
    for (int e = 0; e < E; e++) vec[lane + 64 * e] = o[e];
    if (is_k && Q8) {
        const size_t row = (size_t)hh * max_seq + pos;
#pragma unroll
        for (int e = 0; e < E; e++) {
            q8_store_lane(o[e], lane, e, c8.kq + row * HD, c8.ks + row * (HD / 32));
            q8_store_lane(vv[e], lane, e, c8.vq + row * HD, c8.vs + row * (HD / 32));
        }
    } else if (is_k) {
#pragma unroll
        for (int e = 0; e < E; e++) {
            const size_t off = ((size_t)hh * max_seq + pos) * HD + lane + 64 * e;
            kc[off] = o[e];
            vc[off] = vv[e];
        }
    }
}


// ---------------------------------------------------------------------------
// Causal GQA attention over the fp32 cache, one query head pair per block
// (reference gqa_attn_head_pair_f32, dpuf_engine.c:341-577).
// grid: (M, n_kv, ceil(groups/2)); block 256.
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
// ---------------------------------------------------------------------------


template <int HD>
__global__ __launch_bounds__(256) void k_attn_sc(const float* __restrict__ q, const float* __restrict__ kc,
                                                 const int32_t* __restrict__ pos0p, int M, int n_q, int n_kv,
                                                 int max_seq, float scale, int qt, float* __restrict__ S) {
    constexpr int LD = HD + 4;
    extern __shared__ __align__(16) float sm[];
    float* ks = sm;               // [AS_KC][LD]
    float* qs = ks + AS_KC * LD;  // [32][LD], row r = mi * G + hi
    const int kvh = blockIdx.x, m0 = blockIdx.y * qt, t0 = blockIdx.z * AS_KC, tid = threadIdx.x;
    const int G = n_q / n_kv, R = qt * G;
    const int pos0 = *pos0p;
    const int mlast = (m0 + qt < M ? m0 + qt : M) - 1;
    if (t0 > pos0 + mlast) return;  // no query of the tile reaches these keys
    {
        // every thread's K and q loads are issued before any LDS store
        constexpr int NK = AS_KC * (HD / 4) / 256, NQ = 32 * (HD / 4) / 256;
        float4 kx[NK], qx[NQ];
#pragma unroll
        for (int k = 0; k < NK; k++) {
            const int e = tid + 256 * k, kr = e / (HD / 4), c = e % (HD / 4);
            const int t = t0 + kr < max_seq ? t0 + kr : max_seq - 1;
            kx[k] = *(const float4*)(kc + ((size_t)kvh * max_seq + t) * HD + 4 * c);
        }
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int e = tid + 256 * k, r = e / (HD / 4), c = e % (HD / 4);
            const int mi = r / G, hi = r % G, m = m0 + mi < M ? m0 + mi : M - 1;
            qx[k] = r < R ? *(const float4*)(q + ((size_t)m * n_q + kvh * G + hi) * HD + 4 * c)
                          : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
#pragma unroll
        for (int k = 0; k < NK; k++) {
            const int e = tid + 256 * k, kr = e / (HD / 4), c = e % (HD / 4);
            *(float4*)&ks[kr * LD + 4 * c] = kx[k];
        }
#pragma unroll
        for (int k = 0; k < NQ; k++) {
            const int e = tid + 256 * k, r = e / (HD / 4), c = e % (HD / 4);
            *(float4*)&qs[r * LD + 4 * c] = qx[k];
        }
    }
    __syncthreads();
    const int rp = tid >> 4, kq = tid & 15;
    if (2 * rp >= R) return;
    float acc[2][4][8];
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 4; b++)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[a][b][j] = 0.0f;
    const float* q0 = qs + (2 * rp) * LD;
    const float* q1 = qs + (2 * rp + 1 < R ? 2 * rp + 1 : 2 * rp) * LD;
    // keys kq, kq + 16, kq + 32, kq + 48: adjacent lanes read adjacent K rows
    // (stride LD = 4 mod 32 words), which spreads them over the banks
    const float* k0 = ks + kq * LD;
    for (int i = 0; i < HD; i += 8) {
        float qa[2][8], ka[4][8];
        *(float4*)&qa[0][0] = *(const float4*)(q0 + i);
        *(float4*)&qa[0][4] = *(const float4*)(q0 + i + 4);
        *(float4*)&qa[1][0] = *(const float4*)(q1 + i);
        *(float4*)&qa[1][4] = *(const float4*)(q1 + i + 4);
#pragma unroll
        for (int b = 0; b < 4; b++) {
            *(float4*)&ka[b][0] = *(const float4*)(k0 + 16 * b * LD + i);
            *(float4*)&ka[b][4] = *(const float4*)(k0 + 16 * b * LD + i + 4);
        }
#pragma unroll
        for (int a = 0; a < 2; a++)
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int j = 0; j < 8; j++) acc[a][b][j] = fmaf(qa[a][j], ka[b][j], acc[a][b][j]);
    }
#pragma unroll
    for (int a = 0; a < 2; a++) {
        const int r = 2 * rp + a;
        if (r >= R) continue;
        const int mi = r / G, hi = r % G, m = m0 + mi;
        if (m >= M) continue;
        const int L = pos0 + m + 1, n4 = L & ~3;
        const bool single = (G & 1) && hi == G - 1;
        float* srow = S + ((size_t)m * n_q + kvh * G + hi) * max_seq;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int t = t0 + kq + 16 * b;
            if (t >= L) continue;
            float sc;
            if (t < n4) sc = hsum8_hadd(acc[a][b]);
            else if (!single) sc = hsum8(acc[a][b]);
            else sc = score_dot2(qs + r * LD, ks + (kq + 16 * b) * LD, HD);
            srow[t] = sc * scale;
        }
    }
}


template <int HD, int AP_NT, bool Q8>
__global__ __launch_bounds__(AP_NT) void k_attn_pv(const float* __restrict__ S, const float* __restrict__ vc,
                                                 const int32_t* __restrict__ pos0p, int M, int n_q, int n_kv,
                                                 int max_seq, int qt, int dw, int lcap, int vk,
                                                 float* __restrict__ out, const int8_t* __restrict__ vq,
                                                 const float* __restrict__ vsc) {
    extern __shared__ __align__(16) float sm[];
    __shared__ float part[AP_NT];
    __shared__ float rowv[32][2];  // max, 1 / sum
    const int kvh = blockIdx.x, m0 = blockIdx.y * qt, d0 = blockIdx.z * dw, tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int G = n_q / n_kv, R = qt * G, tpr = AP_NT / R;
    const int pos0 = *pos0p;
    float* P = sm;  // [R][lcap], padded to a multiple of 1024 floats
    float* Vs = sm + ((R * lcap + 1023) & ~1023);  // [2][dw][vk + 4]: a dim's keys contiguous
    const int vld = vk + 4;
    float* scl = Vs + 2 * dw * vld;  // Q8: [2][vk] scales of the chunk's keys
    float* Wq = scl + 2 * vk;        // Q8: [R][vk] weights p * scale
    auto row_len = [&](int r) { return m0 + r / G < M ? pos0 + m0 + r / G + 1 : 0; };
    int Lmax = 0;
    for (int r = 0; r < R; r++) Lmax = row_len(r) > Lmax ? row_len(r) : Lmax;
    // V chunk c -> registers (issued early); registers -> LDS, transposed
    const float* Vh = Q8 ? nullptr : vc + (size_t)kvh * max_seq * HD + d0;
    const int8_t* Vq = Q8 ? vq + (size_t)kvh * max_seq * HD + d0 : nullptr;
    const float* Vsc = Q8 ? vsc + (size_t)kvh * max_seq * (HD / 32) + (d0 >> 5) : nullptr;
    const int nv4 = vk * (dw / 4);  // 4-dim pieces per chunk (1024)
    constexpr int NV = 1024 / AP_NT;
    float4 vreg[NV];
    float sreg[NV];  // Q8: scales of keys tid + AP_NT k of the chunk (vk <= 1024)
    auto v_load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = tid + AP_NT * k, kr = e / (dw / 4), c = e % (dw / 4);
            const bool ok = e < nv4 && c0 + kr < Lmax;
            if (Q8) {
                const uint32_t w = ok ? *(const uint32_t*)(Vq + (size_t)(c0 + kr) * HD + 4 * c) : 0u;
                vreg[k] = make_float4((float)(int8_t)(w & 0xFF), (float)(int8_t)((w >> 8) & 0xFF),
                                      (float)(int8_t)((w >> 16) & 0xFF), (float)(int8_t)(w >> 24));
                sreg[k] = (e < vk && c0 + e < Lmax) ? Vsc[(size_t)(c0 + e) * (HD / 32)] : 0.0f;
            } else {
                vreg[k] = ok ? *(const float4*)(Vh + (size_t)(c0 + kr) * HD + 4 * c)
                             : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    };
    auto v_store = [&](int buf) {
        float* vb = Vs + buf * dw * vld;
#pragma unroll
        for (int k = 0; k < NV; k++) {
            const int e = tid + AP_NT * k, kr = e / (dw / 4), c = e % (dw / 4);
            if (e < nv4) {
                vb[(4 * c + 0) * vld + kr] = vreg[k].x;
                vb[(4 * c + 1) * vld + kr] = vreg[k].y;
                vb[(4 * c + 2) * vld + kr] = vreg[k].z;
                vb[(4 * c + 3) * vld + kr] = vreg[k].w;
            }
            if (Q8 && e < vk) scl[buf * vk + e] = sreg[k];
        }
    };
    v_load(0);
    // score rows -> LDS by direct-to-LDS loads (1 KB per wave instruction,
    // all in flight together; the last one may run into the padding);
    // elements past a row's length are don't-care
    {
        const int n4w = lcap >> 2, tot = R * n4w;
        for (int base = wv * 64; base < tot; base += AP_NT) {
            const int e = base + lane, r = e / n4w, c = e % n4w;
            const int rr = e < tot ? r : 0, mq = m0 + rr / G < M ? m0 + rr / G : M - 1;
            int t = 4 * c;
            if (e >= tot || t + 3 >= max_seq) t = 0;
            const float* src = S + ((size_t)mq * n_q + kvh * G + rr % G) * max_seq + t;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(P + 4 * base), 16, 0, 0);
        }
    }
    v_store(0);
    __syncthreads();
    // row max (tpr threads per row, float4 reads, four running maxima)
    {
        const int r = tid / tpr, j = tid % tpr;
        float m4[4] = {-1e30f, -1e30f, -1e30f, -1e30f};
        if (r < R) {
            const int L = row_len(r), L4 = L & ~3;
            for (int t = 4 * j; t < L4; t += 4 * tpr) {
                const float4 x = *(const float4*)&P[r * lcap + t];
                m4[0] = fmaxf(m4[0], x.x);
                m4[1] = fmaxf(m4[1], x.y);
                m4[2] = fmaxf(m4[2], x.z);
                m4[3] = fmaxf(m4[3], x.w);
            }
            if (j < L - L4) m4[0] = fmaxf(m4[0], P[r * lcap + L4 + j]);
        }
        // when a row's tpr threads are whole waves (tpr a multiple of 64),
        // reduce within the wave first
        float mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
        if (tpr % 64 == 0) {
#pragma unroll
            for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        }
        part[tid] = mx;
    }
    __syncthreads();
    if (tid < R) {
        const int step = tpr % 64 == 0 ? 64 : 1;
        float mx = part[tid * tpr];
        for (int j = step; j < tpr; j += step) mx = fmaxf(mx, part[tid * tpr + j]);
        rowv[tid][0] = mx;
    }
    __syncthreads();
    // exp: the polynomial on t < kv_len & ~7 (float4 at a time), expf on the tail
    {
        const int n4w = lcap >> 2;
        for (int e = tid; e < R * n4w; e += AP_NT) {
            const int r = e / n4w, c = e % n4w, n8 = row_len(r) & ~7;
            if (4 * c >= n8) continue;
            const float mx = rowv[r][0];
            float4 x = *(float4*)&P[r * lcap + 4 * c];
            x.x = exp_poly(x.x - mx);
            x.y = exp_poly(x.y - mx);
            x.z = exp_poly(x.z - mx);
            x.w = exp_poly(x.w - mx);
            *(float4*)&P[r * lcap + 4 * c] = x;
        }
        if (tid < 8 * R) {
            const int r = tid >> 3, L = row_len(r), t = (L & ~7) + (tid & 7);
            if (t < L) P[r * lcap + t] = expf_libc(P[r * lcap + t] - rowv[r][0]);
        }
    }
    __syncthreads();
    // the reference's eight sum lanes, each a chain over t = j (mod 8)
    if (tid < 8 * R) {
        const int r = tid >> 3, j = tid & 7;
        const int n8 = row_len(r) & ~7;
        part[tid] = lds_sum_chain(P + r * lcap + j, 8, n8 >> 3);
    }
    __syncthreads();
    if (tid < R) {
        const int L = row_len(tid), n8 = L & ~7;
        float sp = hsum8(part + 8 * tid);
        for (int t = n8; t < L; t++) sp += P[tid * lcap + t];
        rowv[tid][1] = 1.0f / (sp + 1e-12f);
    }
    __syncthreads();
    // p = e * inv in place (the reference's normalising multiply), once for
    // all the dims' chains
    {
        const int n4w = lcap >> 2;
        for (int e = tid; e < R * n4w; e += AP_NT) {
            const int r = e / n4w, c = e % n4w;
            if (4 * c >= row_len(r)) continue;
            const float inv = rowv[r][1];
            float4 x = *(float4*)&P[r * lcap + 4 * c];
            x.x = x.x * inv;
            x.y = x.y * inv;
            x.z = x.z * inv;
            x.w = x.w * inv;
            *(float4*)&P[r * lcap + 4 * c] = x;
        }
    }
    // P.V: thread (r, d); V chunks double-buffered, the next one loading
    // while the current one is consumed
    const int r = tid / dw, d = tid % dw;
    const bool act = r < R && row_len(r) > 0;
    const int L = act ? row_len(r) : 0;
    // the fp32 single-head path chains nested key pairs; the int8 one does not
    // (dpuf_engine.c:535-558 against 764-778)
    const bool nested = !Q8 && (G & 1) && (r % G) == G - 1 && (HD & 63) == 0;
    const float* prow = Q8 ? Wq + (act ? r : 0) * vk : P + (act ? r : 0) * lcap;
    float a = 0.0f;
    int buf = 0;
    for (int c0 = 0; c0 < Lmax; c0 += vk) {
        const bool more = c0 + vk < Lmax;
        if (more) v_load(c0 + vk);
        __syncthreads();  // chunk c0 in Vs[buf] (and P normalised on the first pass)
        if (Q8) {
            for (int e = tid; e < R * vk; e += AP_NT) {
                const int rr = e / vk, t = e % vk;
                Wq[e] = c0 + t < row_len(rr) ? P[rr * lcap + c0 + t] * scl[buf * vk + t] : 0.0f;
            }
            __syncthreads();
        }
        if (act && c0 < L) {
            const int n = L - c0 < vk ? L - c0 : vk;
            const float* vp = Vs + buf * dw * vld + d * vld;
            const float* pr = Q8 ? prow : prow + c0;
            a = nested ? pv_chain<true>(pr, vp, n, a) : pv_chain<false>(pr, vp, n, a);
        }
        if (Q8) __syncthreads();  // every chain is done with Wq
        if (more) v_store(buf ^ 1);
        buf ^= 1;
    }
    if (act) out[((size_t)(m0 + r / G) * n_q + kvh * G + r % G) * HD + d0 + d] = a;
}


// ---------------------------------------------------------------------------
// k_attn_pvt: softmax and P.V for prefill, register-tiled.  Workgroup (kv
// head, tile of qt = 32 / G queries): R = 32 score rows, all HD dims.  The
// rows come into LDS by direct-to-LDS loads and go through the same softmax
// as k_attn_pv (max; exp polynomial on the 8-aligned part, expf on the tail;
// the reference's eight sum lanes, eng_hsum256 and the tail in order;
// 1 / (sum + 1e-12)), and are normalised in place once (p = e * inv, the
// reference's multiply).  Thread (ri, di) then keeps the 4 x 4 outputs of
// rows ri + 8k (k < 4) and dims 4di .. 4di + 3 in registers and runs each
// output's chain a = fma(p[t], v[t], a) over the keys in order: per 4 keys
// one float4 of p per row from LDS and one float4 of V per key, 64 FMAs.  V
// comes from L2 straight into registers, PVT_KV keys a batch with the next
// batch in flight: the eight lanes of a wave that share a row group hold
// eight consecutive float4 of the key's row, one 128-byte read per wave.
// Keys at or past a row's kv_len (only the tile's last few keys: its rows end
// at consecutive positions) leave that row's chains untouched.  G even (no
// single trailing head), HD in {64, 128, 256}.
// ---------------------------------------------------------------------------
#define PVT_R 32  // score rows per workgroup (a multiple of 8 PVT_RT)
#define PVT_RT 4  // rows per thread in P.V (workgroup of 8 HD / PVT_RT threads)
#define PVT_KV 8  // keys per register batch of V

// p of keys t .. t + 3 for the thread's RT rows (t clamped into the row so a
// read ahead of the last keys stays inside it; such values are not used)
template <int RT>
DEV void pvt_readp(const float* pr, int ldp, int rs, int t, float4 (&p4)[RT]) {
    t = t < ldp - 4 ? t : ldp - 4;
#pragma unroll
    for (int k = 0; k < RT; k++) p4[k] = *(const float4*)(pr + (size_t)k * rs + t);
}

// 4 keys of the tile: rows' p (already read), V from registers
template <int RT>
DEV void pvt_keys4(float (&acc)[RT][4], const float4 (&p4)[RT], const float4* v) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int k = 0; k < RT; k++) {
            const float pk = j == 0 ? p4[k].x : j == 1 ? p4[k].y : j == 2 ? p4[k].z : p4[k].w;
            acc[k][0] = fmaf(pk, v[j].x, acc[k][0]);
            acc[k][1] = fmaf(pk, v[j].y, acc[k][1]);
            acc[k][2] = fmaf(pk, v[j].z, acc[k][2]);
            acc[k][3] = fmaf(pk, v[j].w, acc[k][3]);
        }
    }
}

template <int HD, int RT>
__global__ __launch_bounds__(PVT_R * HD / (4 * RT)) void k_attn_pvt(const float* __restrict__ S, const float* __restrict__ vc,
                                                         const int32_t* __restrict__ pos0p, int M, int n_q, int n_kv,
                                                         int max_seq, int qt, int ldp, float* __restrict__ out,
                                                         const uint8_t* __restrict__ o_sign, DpufPrep op) {
    constexpr int R = PVT_R, NT = R * HD / (4 * RT), KV = PVT_KV;  // (R / RT) row groups x (HD / 4) dim groups
    constexpr int NRG = R / RT;                                     // row groups
    static_assert(R % (8 * RT) == 0 || R == 8 * RT, "whole row bands of 8 row groups");
    constexpr int TPR = NT / R;  // threads per row in the softmax phases
    extern __shared__ __align__(16) float P[];  // [R][ldp]
    __shared__ float part[8 * R];
    __shared__ float rowv[R][2];  // max, 1 / sum
    // query tiles in dispatch order: the later (longer) half descending, then
    // the earlier half ascending, so the two workgroups a CU takes together
    // carry about the same number of keys
    const int ny = gridDim.y, half = (ny + 1) / 2;
    const int ty = (int)blockIdx.y < half ? ny - 1 - (int)blockIdx.y : (int)blockIdx.y - half;
    const int kvh = blockIdx.x, m0 = ty * qt, tid = threadIdx.x;
    const int lane = tid & 63, wv = tid >> 6;
    const int G = n_q / n_kv;
    const int pos0 = *pos0p;
    const int mq = (m0 + qt < M ? m0 + qt : M) - m0;  // queries of this tile
    auto row_len = [&](int r) { return r / G < mq ? pos0 + m0 + r / G + 1 : 0; };
    const int Lmax = pos0 + m0 + mq, Lmin = pos0 + m0 + 1;
    // score rows -> P (row r at r * ldp; 256 floats per wave instruction, ldp
    // >= the rows' length rounded up to 256, so rows never overlap)
    {
        const int nch = (Lmax + 255) >> 8;
        for (int u = wv; u < R * nch; u += NT / 64) {
            const int r = u / nch, ch = u % nch;
            const int rr = r / G < mq ? r : 0;
            int t = 256 * ch + 4 * lane;
            if (t + 3 >= max_seq) t = 0;
            const float* src = S + ((size_t)(m0 + rr / G) * n_q + kvh * G + rr % G) * max_seq + t;
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)(P + (size_t)r * ldp + 256 * ch), 16, 0,
                                             0);
        }
    }
    __syncthreads();
    // row max: TPR consecutive threads per row, four running maxima each
    {
        const int r = tid / TPR, j = tid % TPR;
        float m4[4] = {-1e30f, -1e30f, -1e30f, -1e30f};
        const int L = row_len(r), L4 = L & ~3;
        for (int t = 4 * j; t < L4; t += 4 * TPR) {
            const float4 x = *(const float4*)&P[r * ldp + t];
            m4[0] = fmaxf(m4[0], x.x);
            m4[1] = fmaxf(m4[1], x.y);
            m4[2] = fmaxf(m4[2], x.z);
            m4[3] = fmaxf(m4[3], x.w);
        }
        if (j < L - L4) m4[0] = fmaxf(m4[0], P[r * ldp + L4 + j]);
        float mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
#pragma unroll
        for (int o = TPR / 2; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
        if (j == 0) rowv[r][0] = mx;
    }
    __syncthreads();
    // exp: the polynomial on t < kv_len & ~7 (float4 at a time), expf on the tail
    {
        const int n4w = ldp >> 2;
        for (int e = tid; e < R * n4w; e += NT) {
            const int r = e / n4w, c = e % n4w, n8 = row_len(r) & ~7;
            if (4 * c >= n8) continue;
            const float mx = rowv[r][0];
            float4 x = *(float4*)&P[r * ldp + 4 * c];
            x.x = exp_poly(x.x - mx);
            x.y = exp_poly(x.y - mx);
            x.z = exp_poly(x.z - mx);
            x.w = exp_poly(x.w - mx);
            *(float4*)&P[r * ldp + 4 * c] = x;
        }
        for (int e = tid; e < 8 * R; e += NT) {
            const int r = e >> 3, L = row_len(r), t = (L & ~7) + (e & 7);
            if (t < L) P[r * ldp + t] = expf_libc(P[r * ldp + t] - rowv[r][0]);
        }
    }
    __syncthreads();
    // the reference's eight sum lanes, each a chain over t = j (mod 8)
    for (int e = tid; e < 8 * R; e += NT) {
        const int r = e >> 3, j = e & 7;
        part[e] = lds_sum_chain(P + r * ldp + j, 8, (row_len(r) & ~7) >> 3);
    }
    __syncthreads();
    if (tid < R) {
        const int L = row_len(tid), n8 = L & ~7;
        float sp = hsum8(part + 8 * tid);
        for (int t = n8; t < L; t++) sp += P[tid * ldp + t];
        rowv[tid][1] = 1.0f / (sp + 1e-12f);
    }
    __syncthreads();
    // p = e * inv, in place
    {
        const int n4w = ldp >> 2;
        for (int e = tid; e < R * n4w; e += NT) {
            const int r = e / n4w, c = e % n4w;
            if (4 * c >= row_len(r)) continue;
            const float inv = rowv[r][1];
            float4 x = *(float4*)&P[r * ldp + 4 * c];
            x.x = x.x * inv;
            x.y = x.y * inv;
            x.z = x.z * inv;
            x.w = x.w * inv;
            *(float4*)&P[r * ldp + 4 * c] = x;
        }
    }
    __syncthreads();
    // P.V: a wave holds 8 row groups x 8 dim groups, lane = 8 * (ri % 8) + di % 8
    constexpr int WPR = HD / 32;  // waves per block of 8 row groups
    const int ri = 8 * (wv / WPR) + (lane >> 3), di = 8 * (wv % WPR) + (lane & 7);
    float acc[RT][4];
#pragma unroll
    for (int k = 0; k < RT; k++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[k][i] = 0.0f;
    int Lr[RT];
#pragma unroll
    for (int k = 0; k < RT; k++) Lr[k] = row_len(ri + NRG * k);
    // the thread's rows ri + 8k: the 8 row groups of a wave read rows ldp
    // apart (ldp = 4 mod 64 words), on distinct banks; 4 consecutive rows per
    // thread put them only 4 ldp apart, two to four groups per bank
    const int rs = NRG * ldp;
    const float* pr = P + (size_t)ri * ldp;
    const float* vg = vc + (size_t)kvh * max_seq * HD + 4 * di;
    // keys below Lmin, in whole batches, go to every row unconditionally
    const int nfull = Lmin / KV * KV;
    float4 va[KV], vb[KV];
#pragma unroll
    for (int j = 0; j < KV; j++) va[j] = *(const float4*)(vg + (size_t)(j < max_seq ? j : max_seq - 1) * HD);
    int t0 = 0;
    // (the scheduling barriers keep each batch's V loads ahead of the FMAs of
    // the batch before it, and each 4 keys' p reads ahead of the FMAs of the 4
    // keys before them, so their latencies are covered)
    float4 pa[RT], pb[RT];
    pvt_readp<RT>(pr, ldp, rs, 0, pa);
    for (; t0 + 2 * KV <= nfull; t0 += 2 * KV) {
#pragma unroll
        for (int j = 0; j < KV; j++) {
            const int t = t0 + KV + j;
            vb[j] = *(const float4*)(vg + (size_t)(t < max_seq ? t : max_seq - 1) * HD);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 2 * KV; j += 8) {
            const float4* vv = j < KV ? va + j : vb + (j - KV);
            pvt_readp<RT>(pr, ldp, rs, t0 + j + 4, pb);
            __builtin_amdgcn_sched_barrier(0);
            pvt_keys4<RT>(acc, pa, vv);
            __builtin_amdgcn_sched_barrier(0);
            pvt_readp<RT>(pr, ldp, rs, t0 + j + 8, pa);
            __builtin_amdgcn_sched_barrier(0);
            pvt_keys4<RT>(acc, pb, vv + 4);
            __builtin_amdgcn_sched_barrier(0);
            if (j + 8 == KV) {
#pragma unroll
                for (int jj = 0; jj < KV; jj++) {
                    const int t = t0 + 2 * KV + jj;
                    va[jj] = *(const float4*)(vg + (size_t)(t < max_seq ? t : max_seq - 1) * HD);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    if (t0 + KV <= nfull) {
#pragma unroll
        for (int j = 0; j < KV; j += 4) {
            pvt_readp<RT>(pr, ldp, rs, t0 + j, pa);
            pvt_keys4<RT>(acc, pa, va + j);
        }
        t0 += KV;
    }
    // the tile's last keys: row k takes key t only while t < its kv_len
    for (int t = t0; t < Lmax; t++) {
        const float4 v = *(const float4*)(vg + (size_t)t * HD);
#pragma unroll
        for (int k = 0; k < RT; k++) {
            if (t < Lr[k]) {
                const float pk = pr[(size_t)k * rs + t];
                acc[k][0] = fmaf(pk, v.x, acc[k][0]);
                acc[k][1] = fmaf(pk, v.y, acc[k][1]);
                acc[k][2] = fmaf(pk, v.z, acc[k][2]);
                acc[k][3] = fmaf(pk, v.w, acc[k][3]);
            }
        }
    }
    if (!op.q) {
#pragma unroll
        for (int k = 0; k < RT; k++) {
            const int r = ri + NRG * k;
            if (Lr[k] > 0)
                *(float4*)(out + ((size_t)(m0 + r / G) * n_q + kvh * G + r % G) * HD + 4 * di) =
                    make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
        }
        return;
    }
    // The prep of the O projection's input for the tile's rows (k_prep's
    // arithmetic): the tile goes to LDS (over P, once every thread is done
    // with it), then quad q = (row, 64-column block of the head) takes 16
    // columns per lane through the signs, the FWHT-64 and the quantisation.
    constexpr int LDT = HD + 4;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < RT; k++)
        *(float4*)(P + (size_t)(ri + NRG * k) * LDT + 4 * di) = make_float4(acc[k][0], acc[k][1], acc[k][2], acc[k][3]);
    __syncthreads();
    const int qd = n_q * HD, nb = qd >> 5;
    for (int qq = tid; qq < R * HD / 16; qq += NT) {  // quads of a row never straddle the loop's steps
        const int bi = qq >> 2, qp = qq & 3, r = bi / (HD / 64), bh = bi % (HD / 64);
        if (r / G >= mq) continue;  // whole quads
        float v[16];
        load16(P + (size_t)r * LDT + 64 * bh + 16 * qp, v);
        const int m = m0 + r / G, blk = (kvh * G + r % G) * (HD / 64) + bh;
        apply_sign_bits(v, quad_sign_bits(o_sign, blk, qp));
        quad_fwht64(v, qp);
        quad_quant_store(v, qp, blk, op.q + (size_t)m * qd, op.s + (size_t)m * nb, op.m + (size_t)m * nb,
                         op.h ? op.h + (size_t)m * qd : nullptr);
    }
}

__global__ __launch_bounds__(256) void k_attn(const float* __restrict__ q, const float* __restrict__ kc,
                                              const float* __restrict__ vc, float* __restrict__ out,
                                              float* __restrict__ scores, const int32_t* __restrict__ pos0p,
                                              int n_q, int n_kv, int hd, int max_seq, float scale) {
    extern __shared__ float qs[];  // 2 * hd
    __shared__ float red[2][256];
    __shared__ float vs8[2][8];
    __shared__ float inv_sh[2];
    const int m = blockIdx.x, kvh = blockIdx.y, gp = blockIdx.z, tid = threadIdx.x;
    const int groups = n_q / n_kv;
    const int g0 = 2 * gp;
    const bool pair = (g0 + 1 < groups);
    const int nh = pair ? 2 : 1;
    const int qh0 = kvh * groups + g0;
    const int kv_len = *pos0p + m + 1;
    const float* K = kc + (size_t)kvh * max_seq * hd;
    const float* V = vc + (size_t)kvh * max_seq * hd;
    for (int i = tid; i < nh * hd; i += blockDim.x) qs[i] = q[((size_t)m * n_q + qh0) * hd + i];
    __syncthreads();
    float* sc0 = scores + ((size_t)m * n_q + qh0) * max_seq;
    float* sc1 = sc0 + max_seq;
    const int n4 = kv_len & ~3;
    float mx0 = -1e30f, mx1 = -1e30f;
    for (int t = tid; t < kv_len; t += blockDim.x) {
        const float* kp = K + (size_t)t * hd;
        float s0, s1 = 0.0f;
        if (t < n4) {
            s0 = score_hadd(qs, kp, hd) * scale;
            if (pair) s1 = score_hadd(qs + hd, kp, hd) * scale;
        } else if (pair) {
            s0 = score_hsum(qs, kp, hd) * scale;
            s1 = score_hsum(qs + hd, kp, hd) * scale;
        } else {
            s0 = score_dot2(qs, kp, hd) * scale;
        }
        sc0[t] = s0;
        mx0 = s0 > mx0 ? s0 : mx0;
        if (pair) {
            sc1[t] = s1;
            mx1 = s1 > mx1 ? s1 : mx1;
        }
    }
    red[0][tid] = mx0;
    red[1][tid] = mx1;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (tid < w) {
            red[0][tid] = fmaxf(red[0][tid], red[0][tid + w]);
            red[1][tid] = fmaxf(red[1][tid], red[1][tid + w]);
        }
        __syncthreads();
    }
    const float M0 = red[0][0], M1 = red[1][0];
    const int n8 = kv_len & ~7;
    for (int t = tid; t < kv_len; t += blockDim.x) {
        sc0[t] = t < n8 ? exp_poly(sc0[t] - M0) : expf_libc(sc0[t] - M0);
        if (pair) sc1[t] = t < n8 ? exp_poly(sc1[t] - M1) : expf_libc(sc1[t] - M1);
    }
    __syncthreads();
    if (tid < 16) {
        const int hsel = tid >> 3, j = tid & 7;
        if (hsel < nh) {
            const float* sc = hsel ? sc1 : sc0;
            float a = 0.0f;
            for (int t = j; t < n8; t += 8) a = a + sc[t];
            vs8[hsel][j] = a;
        }
    }
    __syncthreads();
    if (tid < nh) {
        const float* sc = tid ? sc1 : sc0;
        float sp = hsum8(vs8[tid]);
        for (int t = n8; t < kv_len; t++) sp += sc[t];
        inv_sh[tid] = 1.0f / (sp + 1e-12f);
    }
    __syncthreads();
    for (int t = tid; t < kv_len; t += blockDim.x) {
        sc0[t] = sc0[t] * inv_sh[0];
        if (pair) sc1[t] = sc1[t] * inv_sh[1];
    }
    __syncthreads();
    for (int o = tid; o < nh * hd; o += blockDim.x) {
        const int hsel = o / hd, d = o % hd;
        const float* p = hsel ? sc1 : sc0;
        float a = 0.0f;
        if (pair) {
            for (int t = 0; t < kv_len; t++) a = fmaf(p[t], V[(size_t)t * hd + d], a);
        } else if ((hd & 63) == 0) {
            int t = 0;
            for (; t + 1 < kv_len; t += 2)
                a = fmaf(p[t], V[(size_t)t * hd + d], fmaf(p[t + 1], V[(size_t)(t + 1) * hd + d], a));
            if (t < kv_len) a = fmaf(p[t], V[(size_t)t * hd + d], a);
        } else {
            for (int t = 0; t < kv_len; t++) a = fmaf(p[t], V[(size_t)t * hd + d], a);
        }
        out[((size_t)m * n_q + qh0 + hsel) * hd + d] = a;
    }
}

// ---------------------------------------------------------------------------
// Attention over the int8 KV cache (kv_type 1; reference
// gqa_attn_head_pair_q8, dpuf_engine.c:579-752), one workgroup per (token,
// kv head, query-head pair), any M.  Scores: a key of the pair path (keys in
// pairs t, t + 1 while t + 1 < kv_len) keeps 8 lane accumulators, per
// 32-block t = fma(q_lo, k_lo, fma(q_hi, k_hi, t)) over the block's two
// 16-column halves then s = fma(t, k_scale, s), summed by the hadd tree; the
// pair path's last odd key and every key of the single-head path use
// dot_f32_q8_blk32's two accumulators per block and eng_hsum256.  Softmax as
// the fp32 path.  P.V: a = fma(p_k * v_scale[k][block], float(v[k][d]), a),
// keys in order.
// ---------------------------------------------------------------------------
DEV float q8_pair_score(const float* q, const int8_t* kp, const float* ks, int hd) {
    float sa[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < (hd >> 5); b++) {
        const int c0 = 32 * b;
        const int4 kw0 = *(const int4*)(kp + c0), kw1 = *(const int4*)(kp + c0 + 16);
        const int8_t* k0 = (const int8_t*)&kw0;
        const int8_t* k1 = (const int8_t*)&kw1;
        const float sc = ks[b];
#pragma unroll
        for (int L = 0; L < 8; L++) {
            float t = fmaf(q[c0 + L], (float)k0[L], fmaf(q[c0 + 8 + L], (float)k0[8 + L], 0.0f));
            t = fmaf(q[c0 + 16 + L], (float)k1[L], fmaf(q[c0 + 24 + L], (float)k1[8 + L], t));
            sa[L] = fmaf(t, sc, sa[L]);
        }
    }
    return hsum8_hadd(sa);
}

DEV float q8_dot_score(const float* q, const int8_t* kp, const float* ks, int hd) {
    float tot[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < (hd >> 5); b++) {
        const int c0 = 32 * b;
        const int4 kw0 = *(const int4*)(kp + c0), kw1 = *(const int4*)(kp + c0 + 16);
        const int8_t* k0 = (const int8_t*)&kw0;
        const int8_t* k1 = (const int8_t*)&kw1;
        const float sc = ks[b];
#pragma unroll
        for (int L = 0; L < 8; L++) {
            float a0 = fmaf(q[c0 + L], (float)k0[L], 0.0f);
            float a1 = fmaf(q[c0 + 8 + L], (float)k0[8 + L], 0.0f);
            a0 = fmaf(q[c0 + 16 + L], (float)k1[L], a0);
            a1 = fmaf(q[c0 + 24 + L], (float)k1[8 + L], a1);
            tot[L] = fmaf(a0 + a1, sc, tot[L]);
        }
    }
    return hsum8(tot);
}

// Scores over the int8 cache: workgroup (kv head, 64 keys, token); the key
// chunk (int8 rows and scales) and the G query rows in LDS; thread (head,
// key) forms one score with the pair path's or dot_f32_q8_blk32's order.
#define Q8_SCK 64

__global__ __launch_bounds__(256) void k_attn_q8_sc(const float* __restrict__ q, DpufKvQ8 c8,
                                                    float* __restrict__ scores, const int32_t* __restrict__ pos0p,
                                                    int n_q, int n_kv, int hd, int max_seq, float scale) {
    extern __shared__ __align__(16) float sq[];  // [G][hd] q rows, then [Q8_SCK][hd] int8 K, [Q8_SCK][nb] scales
    const int kvh = blockIdx.x, t0 = blockIdx.y * Q8_SCK, m = blockIdx.z, tid = threadIdx.x;
    const int G = n_q / n_kv, nb = hd >> 5;
    const int kv_len = *pos0p + m + 1, n2 = kv_len & ~1;
    if (t0 >= kv_len) return;  // whole workgroup
    int8_t* kl = (int8_t*)(sq + G * hd);
    float* kls = (float*)(kl + Q8_SCK * hd);
    for (int e = tid; e < G * hd / 4; e += 256)
        *(float4*)&sq[4 * e] = *(const float4*)(q + ((size_t)m * n_q + kvh * G) * hd + 4 * e);
    const int8_t* K = c8.kq + (size_t)kvh * max_seq * hd;
    const float* KS = c8.ks + (size_t)kvh * max_seq * nb;
    for (int e = tid; e < Q8_SCK * hd / 16; e += 256) {
        const int t = t0 + (16 * e) / hd;
        *(int4*)(kl + 16 * e) =
            t < kv_len ? *(const int4*)(K + (size_t)t0 * hd + 16 * (size_t)e) : make_int4(0, 0, 0, 0);
    }
    for (int e = tid; e < Q8_SCK * nb; e += 256) {
        const int t = t0 + e / nb;
        kls[e] = t < kv_len ? KS[(size_t)t0 * nb + e] : 0.0f;
    }
    __syncthreads();
    for (int o = tid; o < G * Q8_SCK; o += 256) {
        const int r = o / Q8_SCK, kk = o % Q8_SCK, t = t0 + kk;
        if (t >= kv_len) continue;
        const bool pair = 2 * (r / 2) + 1 < G;  // r belongs to a query-head pair
        const float* qr = sq + r * hd;
        const int8_t* kp = kl + kk * hd;
        const float* ksp = kls + kk * nb;
        const float sc = (pair && t < n2) ? q8_pair_score(qr, kp, ksp, hd) : q8_dot_score(qr, kp, ksp, hd);
        scores[((size_t)m * n_q + kvh * G + r) * max_seq + t] = sc * scale;
    }
}

// One output's chain a = fma(w[t], float(v[t * ld]), a) over n keys of an
// LDS chunk, in key order; 16 keys a batch, the next batch's LDS reads issued
// before the current batch's FMAs so LDS latency stays off the chain.
DEV void q8_pv_load(const float* w, const int8_t* v, int ld, int t, float4 (&wb)[4], int (&vb)[16]) {
#pragma unroll
    for (int i = 0; i < 4; i++) wb[i] = *(const float4*)(w + t + 4 * i);
#pragma unroll
    for (int j = 0; j < 16; j++) vb[j] = v[(t + j) * ld];
}

DEV float q8_pv_fma(const float4 (&wb)[4], const int (&vb)[16], float a) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        a = fmaf(wb[i].x, (float)vb[4 * i], a);
        a = fmaf(wb[i].y, (float)vb[4 * i + 1], a);
        a = fmaf(wb[i].z, (float)vb[4 * i + 2], a);
        a = fmaf(wb[i].w, (float)vb[4 * i + 3], a);
    }
    return a;
}

DEV float q8_pv_chain(const float* w, const int8_t* v, int ld, int n, float a) {
    const int n16 = n & ~15;
    int t = 0;
    if (n16 > 0) {
        float4 wa[4], wc[4];
        int va[16], vc[16];
        q8_pv_load(w, v, ld, 0, wa, va);
        for (t = 0; t + 32 <= n16; t += 32) {
            q8_pv_load(w, v, ld, t + 16, wc, vc);
            __builtin_amdgcn_sched_barrier(0);  // keep the next batch's reads ahead of these FMAs
            a = q8_pv_fma(wa, va, a);
            q8_pv_load(w, v, ld, t + 32 < n16 ? t + 32 : t, wa, va);  // the last reload is unused
            __builtin_amdgcn_sched_barrier(0);
            a = q8_pv_fma(wc, vc, a);
        }
        if (t < n16) {
            a = q8_pv_fma(wa, va, a);
            t += 16;
        }
    }
    for (; t < n; t++) a = fmaf(w[t], (float)v[t * ld], a);
    return a;
}

// Softmax and P.V over the int8 cache, workgroup (token, kv head, pair),
// from the scores k_attn_q8_sc wrote.
__global__ __launch_bounds__(256) void k_attn_q8(DpufKvQ8 c8, float* __restrict__ out, float* __restrict__ scores,
                                                 const int32_t* __restrict__ pos0p, int n_q, int n_kv, int hd,
                                                 int max_seq) {
    extern __shared__ __align__(16) uint8_t lds_q8[];
    __shared__ float red[2][256];
    __shared__ float vs8[2][8];
    __shared__ float inv_sh[2];
    const int m = blockIdx.x, kvh = blockIdx.y, gp = blockIdx.z, tid = threadIdx.x;
    const int groups = n_q / n_kv, nb = hd >> 5;
    const int g0 = 2 * gp;
    const bool pair = (g0 + 1 < groups);
    const int nh = pair ? 2 : 1;
    const int qh0 = kvh * groups + g0;
    const int kv_len = *pos0p + m + 1;
    const int8_t* V = c8.vq + (size_t)kvh * max_seq * hd;
    const float* VS = c8.vs + (size_t)kvh * max_seq * nb;
    float* sc0 = scores + ((size_t)m * n_q + qh0) * max_seq;
    float* sc1 = sc0 + max_seq;
    float mx0 = -1e30f, mx1 = -1e30f;
    for (int t = tid; t < kv_len; t += blockDim.x) {
        const float s0 = sc0[t];
        mx0 = s0 > mx0 ? s0 : mx0;
        if (pair) {
            const float s1 = sc1[t];
            mx1 = s1 > mx1 ? s1 : mx1;
        }
    }
    red[0][tid] = mx0;
    red[1][tid] = mx1;
    __syncthreads();
    for (int w = blockDim.x / 2; w > 0; w >>= 1) {
        if (tid < w) {
            red[0][tid] = fmaxf(red[0][tid], red[0][tid + w]);
            red[1][tid] = fmaxf(red[1][tid], red[1][tid + w]);
        }
        __syncthreads();
    }
    const float M0 = red[0][0], M1 = red[1][0];
    const int n8 = kv_len & ~7;
    for (int t = tid; t < kv_len; t += blockDim.x) {
        sc0[t] = t < n8 ? exp_poly(sc0[t] - M0) : expf_libc(sc0[t] - M0);
        if (pair) sc1[t] = t < n8 ? exp_poly(sc1[t] - M1) : expf_libc(sc1[t] - M1);
    }
    __syncthreads();
    if (tid < 16) {
        const int hsel = tid >> 3, j = tid & 7;
        if (hsel < nh) {
            const float* sc = hsel ? sc1 : sc0;
            float a = 0.0f;
            for (int t = j; t < n8; t += 8) a = a + sc[t];
            vs8[hsel][j] = a;
        }
    }
    __syncthreads();
    if (tid < nh) {
        const float* sc = tid ? sc1 : sc0;
        float sp = hsum8(vs8[tid]);
        for (int t = n8; t < kv_len; t++) sp += sc[t];
        inv_sh[tid] = 1.0f / (sp + 1e-12f);
    }
    __syncthreads();
    for (int t = tid; t < kv_len; t += blockDim.x) {
        sc0[t] = sc0[t] * inv_sh[0];
        if (pair) sc1[t] = sc1[t] * inv_sh[1];
    }
    __syncthreads();
    // P.V over chunks of ck keys staged in LDS: the chunk's int8 V rows and,
    // per (head, key, block), the weight w = p * v_scale (the reference's
    // p * vs product, formed once per chunk instead of once per dim); the next
    // chunk's V and scales are read into registers while this one's chains
    // run.  Thread (head, dim) then runs a = fma(w, float(v), a) in key order.
    const int ck = 32768 / hd;                 // keys per chunk: 32 KB of V
    int8_t* vl = (int8_t*)lds_q8;              // [2][ck][hd]
    float* wl = (float*)(vl + 2 * ck * hd);    // [2][2][nb][ck]
    constexpr int VR = 8;                      // 16-byte V loads per thread per chunk
    int4 vr[VR];
    float4 sr;
    const int vper = ck * hd / 16;             // 16-byte pieces of a V chunk (2048)
    const int sper = ck * nb / 4;              // float4 of its scales
    auto ld = [&](int c0) {
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = tid + 256 * k;
            const int t = c0 + (16 * e) / hd;
            vr[k] = e < vper && t < kv_len ? *(const int4*)(V + (size_t)c0 * hd + 16 * (size_t)e)
                                           : make_int4(0, 0, 0, 0);
        }
        // 4 (key, block) scales per thread; keys past kv_len are not read
        float sv4[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int e = 4 * tid + i;
            sv4[i] = tid < sper && c0 + e / nb < kv_len ? VS[(size_t)c0 * nb + e] : 0.0f;
        }
        sr = make_float4(sv4[0], sv4[1], sv4[2], sv4[3]);
    };
    auto st = [&](int buf, int c0) {
        int8_t* vb = vl + (size_t)buf * ck * hd;
#pragma unroll
        for (int k = 0; k < VR; k++) {
            const int e = tid + 256 * k;
            if (e < vper) *(int4*)(vb + 16 * e) = vr[k];
        }
        // weights from the scales just read: element 4 tid + i is (key, block)
        float* wb = wl + (size_t)buf * 2 * nb * ck;
        if (tid < sper) {
            const float sv[4] = {sr.x, sr.y, sr.z, sr.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = 4 * tid + i, tk = e / nb, b = e % nb;
                if (c0 + tk < kv_len) {
                    wb[b * ck + tk] = sc0[c0 + tk] * sv[i];
                    if (pair) wb[(nb + b) * ck + tk] = sc1[c0 + tk] * sv[i];
                }
            }
        }
    };
    const int o0 = tid, o1 = tid + 256;  // up to two outputs per thread (2 x 256 dims)
    float acc0 = 0.0f, acc1 = 0.0f;
    ld(0);
    st(0, 0);
    __syncthreads();
    int buf = 0;
    for (int c0 = 0; c0 < kv_len; c0 += ck) {
        const bool more = c0 + ck < kv_len;
        if (more) ld(c0 + ck);
        const int n = kv_len - c0 < ck ? kv_len - c0 : ck;
        const int8_t* vb = vl + (size_t)buf * ck * hd;
        const float* wb = wl + (size_t)buf * 2 * nb * ck;
        if (o0 < nh * hd) {
            const int hsel = o0 / hd, d = o0 % hd;
            acc0 = q8_pv_chain(wb + (size_t)(hsel * nb + (d >> 5)) * ck, vb + d, hd, n, acc0);
        }
        if (o1 < nh * hd) {
            const int hsel = o1 / hd, d = o1 % hd;
            acc1 = q8_pv_chain(wb + (size_t)(hsel * nb + (d >> 5)) * ck, vb + d, hd, n, acc1);
        }
        __syncthreads();  // every chain is done with buffer buf ^ 1's last use
        if (more) st(buf ^ 1, c0 + ck);
        __syncthreads();
        buf ^= 1;
    }
    if (o0 < nh * hd) out[((size_t)m * n_q + qh0) * hd + o0] = acc0;
    if (o1 < nh * hd) out[((size_t)m * n_q + qh0) * hd + o1] = acc1;
}

// Rows of fp32 K and V (n rows of HD, one wave per row and tensor) into the
// int8 cache at rows row0 .. row0 + n - 1 (KV injection), and back out as
// q * scale.
template <int HD>
__global__ __launch_bounds__(64) void k_q8_rows(const float* __restrict__ k, const float* __restrict__ v, int n,
                                                DpufKvQ8 c8, size_t row0) {
    const int r = blockIdx.x, lane = threadIdx.x, which = blockIdx.y;
    if (r >= n) return;
    const float* src = (which ? v : k) + (size_t)r * HD;
    int8_t* dst = (which ? c8.vq : c8.kq) + (row0 + r) * HD;
    float* sdst = (which ? c8.vs : c8.ks) + (row0 + r) * (HD / 32);
#pragma unroll
    for (int e = 0; e < HD / 64; e++) q8_store_lane(src[lane + 64 * e], lane, e, dst, sdst);
}

__global__ void k_q8_dequant(DpufKvQ8 c8, size_t off, size_t n, float* __restrict__ k, float* __restrict__ v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        k[i] = (float)c8.kq[off + i] * c8.ks[(off + i) >> 5];
        v[i] = (float)c8.vq[off + i] * c8.vs[(off + i) >> 5];
    }
}


// Attention launches enqueued per path, process-wide (dpuf_amd_attn_path_count).
static int64_t g_attn_paths[DPUF_HIP_ATTN_PATHS];

void attn_path_note(int which) {
    if (which >= 0 && which < DPUF_HIP_ATTN_PATHS) __atomic_fetch_add(&g_attn_paths[which], 1, __ATOMIC_RELAXED);
}

extern "C" {

int64_t dpuf_hip_attn_path_count(int32_t which) {
    if (which < 0 || which >= DPUF_HIP_ATTN_PATHS) return -1;
    return __atomic_load_n(&g_attn_paths[which], __ATOMIC_RELAXED);
}

void dpuf_hip_qk_rope_kv(void* s, int32_t M, float* q, float* k, const float* v, const float* q_norm,
                         const float* k_norm, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                         float* vc, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                         const DpufKvQ8* c8) {
    const dim3 gw((M * (n_q + n_kv) + 3) / 4);
    DpufKvQ8 z;
    memset(&z, 0, sizeof z);
    const DpufKvQ8 c = c8 ? *c8 : z;
#define QKR(HDV)                                                                                                  \
    do {                                                                                                          \
        if (c8)                                                                                                   \
            hipLaunchKernelGGL((k_qk_rope_kv_w<HDV, true>), gw, dim3(256), 0, ST(s), q, k, v, q_norm, k_norm, eps,  \
                               cos_tab, sin_tab, kc, vc, pos0, M, n_q, n_kv, max_seq, c);                         \
        else                                                                                                      \
            hipLaunchKernelGGL((k_qk_rope_kv_w<HDV, false>), gw, dim3(256), 0, ST(s), q, k, v, q_norm, k_norm, eps, \
                               cos_tab, sin_tab, kc, vc, pos0, M, n_q, n_kv, max_seq, c);                         \
    } while (0)
    if (hd == 64) QKR(64);
    else if (hd == 128) QKR(128);
    else if (hd == 256) QKR(256);
    else note(hipErrorInvalidValue, "dpuf_hip_qk_rope_kv: head dim must be 64, 128 or 256");
#undef QKR
    LAUNCHED("k_qk_rope_kv");
}

// Split attention (k_attn_sc + k_attn_pv) over keys up to lmax = pos0 + M
// (or max_seq when the launch is captured for replay at any position).
// Returns -1 without launching when the shape does not fit (group > 32, head
// dim not 64/128/256, or a tile's probabilities not fitting in LDS).
// rope (one-token steps only): the QK-norm, RoPE and KV store ride in the
// scores launch; -1 with nothing launched when the one-token wide path does
// not apply.  wm (or NULL): weight groups the one-token wide path's P.V
// launch warms on the CUs its chain workgroups leave idle.
static int32_t attn_split(void* s, int32_t M, int32_t lmax, const float* q, const float* kc, const float* vc,
                          float* out, float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd,
                          int32_t max_seq, float scale, const uint8_t* o_sign, DpufPrep op, int32_t* prepped,
                          const ScRope* rope, const DpufWarm* wm) {
    if (prepped) *prepped = 0;
    if (rope && M != 1) return -1;
    if (n_kv <= 0 || n_q % n_kv || n_q / n_kv > 32 || (hd != 64 && hd != 128 && hd != 256)) return -1;
    if (lmax > max_seq) lmax = max_seq;
    const int G = n_q / n_kv;
    // scores: up to 32 q rows (queries x group heads) per workgroup
    const int qt1 = 32 / G < M ? 32 / G : M;
    const dim3 g1(n_kv, (M + qt1 - 1) / qt1, (lmax + AS_KC - 1) / AS_KC);
    const size_t lds1 = (size_t)(AS_KC + 32) * (hd + 4) * 4;
    // prefill with an even group: the register-tiled softmax + P.V kernel
    if (M > 1 && (G & 1) == 0 && PVT_R % G == 0) {
        const int ldp = 256 * ((lmax + 255) / 256) + 4;
        const size_t ldst = (size_t)PVT_R * ldp * 4;
        if (ldst <= 150 * 1024) {
            const int qt = PVT_R / G;
            const dim3 gt(n_kv, (M + qt - 1) / qt);
            // the O input prep rides along when asked for (op.q set)
            DpufPrep fop = op;
            if (!prepped) fop.q = NULL;
            if (fop.q) *prepped = 1;
            if (hd == 64) {
                hipLaunchKernelGGL(k_attn_sc<64>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq,
                                   scale, qt1, scores);
                hipLaunchKernelGGL((k_attn_pvt<64, PVT_RT>), gt, dim3(PVT_R * 64 / (4 * PVT_RT)), ldst, ST(s), scores, vc,
                                   pos0p, M, n_q, n_kv, max_seq, qt, ldp, out, o_sign, fop);
            } else if (hd == 128) {
                hipLaunchKernelGGL(k_attn_sc<128>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq,
                                   scale, qt1, scores);
                hipLaunchKernelGGL((k_attn_pvt<128, PVT_RT>), gt, dim3(PVT_R * 128 / (4 * PVT_RT)), ldst, ST(s), scores, vc,
                                   pos0p, M, n_q, n_kv, max_seq, qt, ldp, out, o_sign, fop);
            } else {
                hipLaunchKernelGGL(k_attn_sc<256>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq,
                                   scale, qt1, scores);
                hipLaunchKernelGGL((k_attn_pvt<256, PVT_RT>), gt, dim3(PVT_R * 256 / (4 * PVT_RT)), ldst, ST(s), scores, vc,
                                   pos0p, M, n_q, n_kv, max_seq, qt, ldp, out, o_sign, fop);
            }
            LAUNCHED("k_attn_split_tiled");
            attn_path_note(0);
            return 0;
        }
    }
    // one-token decode with an even group: softmax once per row, then the
    // wide P.V (one wave per kv head and 4 dims); its probabilities stay in
    // global memory, so the LDS budget below does not limit it
    if (M == 1 && attn_wide_f32(s, lmax, q, kc, vc, out, scores, pos0p, n_q, n_kv, hd, max_seq, scale, rope, wm) == 0)
        return 0;
    if (rope) return -1;
    // softmax + P.V in LDS: R = qt2 * G rows of lcap probabilities; about 8
    // rows per workgroup keeps >= 32 dims per P.V chain group, so the
    // softmax each dim chunk repeats stays small next to P.V
    const int lcap = (lmax + 7) & ~7;
    const size_t budget = 112 * 1024;
    int qt2 = 8 / G > 1 ? 8 / G : 1;
    if (qt2 > M) qt2 = M;
    while (qt2 > 1 && (size_t)qt2 * G * lcap * 4 > budget) qt2--;
    if ((size_t)qt2 * G * lcap * 4 > budget) return -1;
    const int R = qt2 * G;
    int dc = 1;
    while (dc < hd / 4 && R * (hd / dc) > 256) dc *= 2;
    const int tiles = n_kv * ((M + qt2 - 1) / qt2);
    while (dc < hd / 4 && tiles * dc < 128) dc *= 2;  // enough workgroups to spread the V reads
    const int dw = hd / dc;
    const int vk = 4096 / dw;  // V chunk: 16 KB (+ padding), two buffers
    const size_t lds2 = ((((size_t)R * lcap + 1023) & ~(size_t)1023) + 2 * (size_t)(vk + 4) * dw) * 4;
    const dim3 g2(n_kv, (M + qt2 - 1) / qt2, dc);
    // 1024 threads for launches of few workgroups (decode: the softmax phases
    // go 4x wider), 256 when many workgroups already fill the chip (prefill)
    const bool wide = (size_t)g2.x * g2.y * g2.z < 1024;
    const dim3 b2(wide ? 1024 : 256);
    if (hd == 64) {
        hipLaunchKernelGGL(k_attn_sc<64>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq, scale,
                           qt1, scores);
        if (wide)
            hipLaunchKernelGGL((k_attn_pv<64, 1024, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q, n_kv,
                               max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
        else
            hipLaunchKernelGGL((k_attn_pv<64, 256, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q, n_kv,
                               max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
    } else if (hd == 128) {
        hipLaunchKernelGGL(k_attn_sc<128>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq, scale,
                           qt1, scores);
        if (wide)
            hipLaunchKernelGGL((k_attn_pv<128, 1024, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q,
                               n_kv, max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
        else
            hipLaunchKernelGGL((k_attn_pv<128, 256, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q,
                               n_kv, max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
    } else {
        hipLaunchKernelGGL(k_attn_sc<256>, g1, dim3(256), lds1, ST(s), q, kc, pos0p, M, n_q, n_kv, max_seq, scale,
                           qt1, scores);
        if (wide)
            hipLaunchKernelGGL((k_attn_pv<256, 1024, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q,
                               n_kv, max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
        else
            hipLaunchKernelGGL((k_attn_pv<256, 256, false>), g2, b2, lds2, ST(s), scores, vc, pos0p, M, n_q,
                               n_kv, max_seq, qt2, dw, lcap, vk, out, nullptr, nullptr);
    }
    LAUNCHED("k_attn_split");
    attn_path_note(2);
    return 0;
}

int32_t dpuf_hip_attn_split(void* s, int32_t M, int32_t lmax, const float* q, const float* kc, const float* vc,
                            float* out, float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd,
                            int32_t max_seq, float scale, const uint8_t* o_sign, DpufPrep op, int32_t* prepped) {
    return attn_split(s, M, lmax, q, kc, vc, out, scores, pos0p, n_q, n_kv, hd, max_seq, scale, o_sign, op, prepped,
                      NULL, NULL);
}

int32_t dpuf_hip_attn_decode_rope(void* s, int32_t lmax, float* q, const float* k, const float* v, const float* qn,
                                  const float* kn, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                                  float* vc, float* out, float* scores, const int32_t* pos0p, int32_t n_q,
                                  int32_t n_kv, int32_t hd, int32_t max_seq, float scale, const DpufWarm* warm) {
    const ScRope r = {k, v, qn, kn, eps, cos_tab, sin_tab, kc, vc};
    DpufPrep none;
    memset(&none, 0, sizeof none);
    return attn_split(s, 1, lmax, q, kc, vc, out, scores, pos0p, n_q, n_kv, hd, max_seq, scale, NULL, none, NULL, &r,
                      warm);
}

void dpuf_hip_attn(void* s, int32_t M, const float* q, const float* kc, const float* vc, float* out, float* scores,
                   const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq, float scale) {
    const int groups = n_q / n_kv;
    hipLaunchKernelGGL(k_attn, dim3(M, n_kv, (groups + 1) / 2), dim3(256), (size_t)2 * hd * sizeof(float), ST(s), q,
                       kc, vc, out, scores, pos0, n_q, n_kv, hd, max_seq, scale);
    LAUNCHED("k_attn");
    attn_path_note(3);
}

void dpuf_hip_attn_q8(void* s, int32_t M, int32_t lmax, const float* q, DpufKvQ8 c8, float* out, float* scores,
                      const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq, float scale,
                      const DpufWarm* warm) {
    const int G = n_q / n_kv;
    if (lmax > max_seq) lmax = max_seq;
    const size_t lds1 = (size_t)G * hd * 4 + (size_t)Q8_SCK * hd + (size_t)Q8_SCK * (hd / 32) * 4;
    hipLaunchKernelGGL(k_attn_q8_sc, dim3(n_kv, (lmax + Q8_SCK - 1) / Q8_SCK, M), dim3(256), lds1, ST(s), q, c8,
                       scores, pos0, n_q, n_kv, hd, max_seq, scale);
    // one token, groups of 2, 4 or 8: the softmax once per row and P.V on one
    // chain wave per (kv head, 4 dims), as for the fp32 cache, with W = p *
    // v_scale and V widened in the producers
    if (M == 1 && attn_wide_q8(s, lmax, pos0, n_q, n_kv, hd, max_seq, scores, out, c8, warm) == 0) {
        attn_path_note(5);
        return;
    }
    // softmax + P.V: the split kernel (as the fp32 cache's) when its tile of
    // probability rows fits in LDS, each dim chunk inside one 32-column block
    const int lcap = (lmax + 7) & ~7;
    const size_t budget = 112 * 1024;
    int qt2 = 8 / G > 1 ? 8 / G : 1;
    if (qt2 > M) qt2 = M;
    while (qt2 > 1 && (size_t)qt2 * G * lcap * 4 > budget) qt2--;
    if (G <= 32 && (size_t)qt2 * G * lcap * 4 <= budget) {
        const int R = qt2 * G;
        int dc = 1;
        while (dc < hd / 4 && R * (hd / dc) > 256) dc *= 2;
        const int tiles = n_kv * ((M + qt2 - 1) / qt2);
        while (dc < hd / 4 && tiles * dc < 128) dc *= 2;
        while (hd / dc > 32) dc *= 2;
        const int dw = hd / dc, vk = 4096 / dw;
        const size_t lds2 = ((((size_t)R * lcap + 1023) & ~(size_t)1023) + 2 * (size_t)(vk + 4) * dw +
                             2 * (size_t)vk + (size_t)R * vk) * 4;
        const dim3 g2(n_kv, (M + qt2 - 1) / qt2, dc);
        const bool wide = (size_t)g2.x * g2.y * g2.z < 1024;
#define PVQ(HDV, NT)                                                                                              \
    hipLaunchKernelGGL((k_attn_pv<HDV, NT, true>), g2, dim3(NT), lds2, ST(s), scores, nullptr, pos0, M, n_q, n_kv, \
                       max_seq, qt2, dw, lcap, vk, out, c8.vq, c8.vs)
        if (lds2 <= 160 * 1024) {
            if (hd == 64) { if (wide) PVQ(64, 1024); else PVQ(64, 256); }
            else if (hd == 128) { if (wide) PVQ(128, 1024); else PVQ(128, 256); }
            else { if (wide) PVQ(256, 1024); else PVQ(256, 256); }
            LAUNCHED("k_attn_q8_sc/k_attn_pv<q8>");
            attn_path_note(5);
            return;
        }
#undef PVQ
    }
    // rows too long for LDS: softmax in memory, P.V per (token, kv head, pair)
    const size_t lds2 = 2 * 32768 + (size_t)2 * 2 * (hd / 32) * (32768 / hd) * 4;
    hipLaunchKernelGGL(k_attn_q8, dim3(M, n_kv, (G + 1) / 2), dim3(256), lds2, ST(s), c8, out, scores, pos0,
                       n_q, n_kv, hd, max_seq);
    LAUNCHED("k_attn_q8_sc/k_attn_q8");
    attn_path_note(5);
}

void dpuf_hip_q8_rows(void* s, const float* k, const float* v, int32_t n, int32_t hd, DpufKvQ8 c8, size_t row0) {
    if (n <= 0) return;
    const dim3 g(n, 2);
    if (hd == 64) hipLaunchKernelGGL(k_q8_rows<64>, g, dim3(64), 0, ST(s), k, v, n, c8, row0);
    else if (hd == 128) hipLaunchKernelGGL(k_q8_rows<128>, g, dim3(64), 0, ST(s), k, v, n, c8, row0);
    else if (hd == 256) hipLaunchKernelGGL(k_q8_rows<256>, g, dim3(64), 0, ST(s), k, v, n, c8, row0);
    else note(hipErrorInvalidValue, "dpuf_hip_q8_rows: head dim must be 64, 128 or 256");
    LAUNCHED("k_q8_rows");
}

void dpuf_hip_q8_dequant(void* s, DpufKvQ8 c8, size_t off, size_t n, float* k, float* v) {
    if (n == 0) return;
    const size_t blocks = (n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096;
    hipLaunchKernelGGL(k_q8_dequant, dim3((unsigned)blocks), dim3(256), 0, ST(s), c8, off, n, k, v);
    LAUNCHED("k_q8_dequant");
}


}  // extern "C"
