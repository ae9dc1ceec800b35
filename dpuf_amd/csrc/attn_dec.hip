// attn_dec.hip -- the fused one-token decode attention (k_attn_dec) with the
// cache warm-up workgroups that run beside it.
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
#include "dev_exp.h"
#include "attn_common.h"

// ---------------------------------------------------------------------------
// Decode attention (M == 1), one workgroup (4 waves) per (kv head,
// query-head pair): QK-norm + NeoX RoPE of the pair's queries and of the new
// key, the KV-cache store of position pos (pair 0 only), causal attention
// over [0, pos], and the prep of the O projection's input for the pair's
// 2 * HD columns.
//
// Arithmetic follows gqa_attn_head_pair_f32 (dpuf_engine.c:341-577) term by
// term.  A score's 8 lane-accumulators (accumulator j: elements j, j+8, ...,
// in order) are split over 2 lanes (lane h holds accumulators 4h .. 4h+3, fed
// by float4 loads of elements 8i + 4h), and the reference's hadd / hsum trees
// are evaluated on them with the same pairings.  Then the exp polynomial with
// the libm expf tail, the 8-lane softmax sum and the per-output P.V chains.
//
// Latency: the K rows of the first ATT_KEYS positions are loaded into
// registers and the first V_ROWS rows of V are copied straight into LDS
// (global_load_lds, 1 KB per wave instruction) at kernel entry, so both
// streams are in flight while the norms and RoPE run.
// ---------------------------------------------------------------------------
#define ATT_KEYS 128  // keys per pass: 2 lanes per key, 256 threads




template <int HD>
__global__ __launch_bounds__(256) void k_attn_dec(const float* __restrict__ q, const float* __restrict__ k,
                                                  const float* __restrict__ v, const float* __restrict__ qn,
                                                  const float* __restrict__ kn, float eps,
                                                  const float* __restrict__ cos_tab, const float* __restrict__ sin_tab,
                                                  float* __restrict__ kc, float* __restrict__ vc,
                                                  const int32_t* __restrict__ pos0p, int n_q, int n_kv, int max_seq,
                                                  float scale,
                                                  float* __restrict__ ao, const uint8_t* __restrict__ o_sign,
                                                  DpufPrep op, float* const* kcs, float* const* vcs, size_t l_off,
                                                  DpufWarm warm) {
    constexpr int V_ROWS = 16384 / HD;  // 64 KB of V rows per LDS chunk
    {
        // workgroups past the query pairs warm the caches for the next launch
        const int ny = (n_q / n_kv + 1) / 2;
        if ((int)blockIdx.y >= ny) {
            warm_read(warm, ((int)blockIdx.y - ny) * (int)gridDim.x + (int)blockIdx.x,
                      (int)(blockIdx.y * gridDim.x + blockIdx.x), threadIdx.x, 256);
            return;
        }
    }
    // token blockIdx.z of a multi-session step: its own q/k/v rows, position
    // and output rows, and (kcs set) its own session's KV cache
    {
        const int mt = blockIdx.z;
        if (kcs) {
            kc = kcs[mt] + l_off;
            vc = vcs[mt] + l_off;
        }
        q += (size_t)mt * n_q * HD;
        k += (size_t)mt * n_kv * HD;
        v += (size_t)mt * n_kv * HD;
        ao += (size_t)mt * n_q * HD;
        pos0p += mt;
        const size_t qd = (size_t)n_q * HD;
        op.q += mt * qd;
        op.s += mt * (qd >> 5);
        op.m += mt * (qd >> 5);
        if (op.h) op.h += mt * qd;
    }
    constexpr int NI = HD / 8;          // float4 steps per key and lane
    constexpr int half = HD / 2;
    extern __shared__ float sm[];
    float* vst = sm;                    // [V_ROWS][HD], 1 KB aligned
    float* qs = vst + V_ROWS * HD;      // [2][HD]
    float* ks = qs + 2 * HD;            // [HD]
    float* vn = ks + HD;                // [HD]
    float* aout = vn + HD;              // [2][HD]
    float* scl = aout + 2 * HD;         // [max(2 * DPUF_HIP_DEC_MAX_KEYS, 3 * HD)]
    __shared__ float part[3][8];
    __shared__ float vs8[2][8];
    __shared__ uint64_t etab[32];  // the expf table (read by the softmax tails)
    const int kvh = blockIdx.x, gp = blockIdx.y, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int groups = n_q / n_kv, g0 = 2 * gp;
    const bool pair = (g0 + 1 < groups);
    const int nh = pair ? 2 : 1;
    const int qh0 = kvh * groups + g0;
    const float* Kc = kc + (size_t)kvh * max_seq * HD;
    const float* Vc = vc + (size_t)kvh * max_seq * HD;

    // V rows [c0, c0 + rows) -> vst, 1 KB per wave instruction (whole
    // instructions: a few rows past the end may come along); rows past the
    // cache end are redirected to row 0 (never read back).
    auto stage_v = [&](int c0, int rows) {
        const int n_ins = (rows * HD + 255) / 256;
        for (int ii = wave; ii < n_ins; ii += 4) {
            const int e = ii * 256 + lane * 4;  // float index inside the chunk
            int t = c0 + e / HD;
            if (t >= max_seq) t = 0;
            __builtin_amdgcn_global_load_lds((const void*)(Vc + (size_t)t * HD + (e % HD)),
                                             (lds_ptr_t)(vst + ii * 256), 16, 0, 0);
        }
    };
    // key kq (one per lane pair) of each pass; lane h holds elements 8i + 4h
    // .. +3.  Rows clamped into the cache, read through a global pointer (the
    // cache base may come from kcs[], and loads through a generic pointer
    // would wait for the V-row LDS DMA before each one).  Keys at or past pos
    // only feed scores that are never stored; key pos itself is replaced by
    // the new key.
    const int kq = tid >> 1, h = tid & 1;
    float4 kr[NI];
    auto load_k = [&](int t0) {
        const int t = min(t0 + kq, max_seq - 1);
        const __attribute__((address_space(1))) gm_f4* kp =
            (const __attribute__((address_space(1))) gm_f4*)(Kc + (size_t)t * HD + 4 * h);
#pragma unroll
        for (int i = 0; i < NI; i++) {
            const gm_f4 x = kp[2 * i];
            kr[i] = make_float4(x[0], x[1], x[2], x[3]);
        }
    };
    // The first pass's K rows and the first chunk of V rows are requested
    // before the position is known, so their round trip overlaps the
    // position's and the q / k / v loads'.
    stage_v(0, V_ROWS);
    load_k(0);
    const uint64_t etab_w = c_exp2_tab[tid & 31];  // to LDS with the first stores below

    // Thread tid owns normalised elements e = tid + 256 * r of [q0 | q1 | k].
    constexpr int NE = (3 * HD + 255) / 256;
    float xe[NE], we[NE];
#pragma unroll
    for (int r = 0; r < NE; r++) {
        const int e = tid + 256 * r, vi = e / HD, i = e % HD;
        xe[r] = 0.0f;
        we[r] = 1.0f;
        if (e < 3 * HD && (vi != 1 || pair)) {
            xe[r] = vi == 2 ? k[(size_t)kvh * HD + i] : q[(size_t)(qh0 + vi) * HD + i];
            const float* nw = vi == 2 ? kn : qn;
            if (nw) we[r] = nw[i];
        }
    }
    constexpr int NV = (HD + 255) / 256;
    float vv0[NV];
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = tid + 256 * r;
        vv0[r] = i < HD ? v[(size_t)kvh * HD + i] : 0.0f;
    }
    // the O input's sign bits of this lane's columns in the prep below:
    // block b = wave + 4 k of the pair's nh * HD / 64, column lane
    constexpr int NPB = (2 * HD / 64 + 3) / 4;
    uint32_t osb = 0;
#pragma unroll
    for (int k = 0; k < NPB; k++) {
        const int b = wave + 4 * k;
        if (o_sign && b < nh * HD / 64) osb |= ((o_sign[8 * ((qh0 * HD) / 64 + b) + (lane >> 3)] >> (lane & 7)) & 1u) << k;
    }
    const int pos = *pos0p;
    const int kv_len = pos + 1;

    // RoPE table entries of the owned elements
    const float* c_row = cos_tab + (size_t)pos * half;
    const float* s_row = sin_tab + (size_t)pos * half;
    float ce[NE], se[NE];
#pragma unroll
    for (int r = 0; r < NE; r++) {
        const int i = (tid + 256 * r) % HD, j = i < half ? i : i - half;
        ce[r] = c_row[j];
        se[r] = s_row[j];
    }

    if (tid < 32) etab[tid] = etab_w;
    float* tmp = scl;  // [3][HD] normalised vectors, before the scores use this space
#pragma unroll
    for (int r = 0; r < NE; r++) {
        const int e = tid + 256 * r;
        if (e < 3 * HD) tmp[e] = xe[r];
    }
#pragma unroll
    for (int r = 0; r < NV; r++) {
        const int i = tid + 256 * r;
        if (i < HD) vn[i] = vv0[r];
    }
    __syncthreads();
    // QK-norm (rms_norm_f32 over hd: 8 FMA lanes + hsum tree), vectors 0 = q0, 1 = q1, 2 = k
    if (tid < 24) {
        const int vi = tid >> 3, jj = tid & 7;
        const float* vec = tmp + vi * HD;
        const float* nw = vi == 2 ? kn : qn;
        if ((vi != 1 || pair) && nw) {
            // all of the lane's elements into registers, then the chain
            float xv[HD / 8];
#pragma unroll
            for (int i = 0; i < HD / 8; i++) xv[i] = vec[jj + 8 * i];
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < HD / 8; i++) a = fmaf(xv[i], xv[i], a);
            part[vi][jj] = a;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NE; r++) {
        const int e = tid + 256 * r, vi = e / HD;
        if (e < 3 * HD && (vi != 1 || pair) && (vi == 2 ? kn : qn)) {
            const float inv = 1.0f / sqrtf(hsum8(part[vi]) / (float)HD + eps);
            tmp[e] = (xe[r] * inv) * we[r];
        }
    }
    __syncthreads();
    // NeoX RoPE (apply_rope_neox_f32, dpuf_engine.c:274-295)
#pragma unroll
    for (int r = 0; r < NE; r++) {
        const int e = tid + 256 * r, vi = e / HD, i = e % HD;
        if (e >= 3 * HD || (vi == 1 && !pair)) continue;
        const float* x = tmp + vi * HD;
        float o;
        if (i < half) o = fmaf(x[i], ce[r], -(x[i + half] * se[r]));
        else o = fmaf(x[i], ce[r], x[i - half] * se[r]);
        if (vi == 2) ks[i] = o;
        else qs[vi * HD + i] = o;
    }
    __syncthreads();
    if (gp == 0) {
        for (int i = tid; i < HD; i += 256) {
            // global stores (kc / vc may come from kcs[] / vcs[])
            ((__attribute__((address_space(1))) float*)kc)[((size_t)kvh * max_seq + pos) * HD + i] = ks[i];
            ((__attribute__((address_space(1))) float*)vc)[((size_t)kvh * max_seq + pos) * HD + i] = vn[i];
        }
    }

    // scores
    // score rows in LDS (kv_len <= DPUF_HIP_DEC_MAX_KEYS, the launch contract)
    float* sc0 = scl;
    float* sc1 = scl + DPUF_HIP_DEC_MAX_KEYS;
    const int n4 = kv_len & ~3;
    for (int t0 = 0; t0 < kv_len; t0 += ATT_KEYS) {
        if (t0 > 0) load_k(t0);
        const int t = t0 + kq;
        if (t == pos) {
#pragma unroll
            for (int i = 0; i < NI; i++) kr[i] = *(const float4*)(ks + 8 * i + 4 * h);
        }
        // accumulators 4h .. 4h+3 of both heads
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f}, b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        float c[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // single-head tail: dot_f32_avx2's second accumulator
        const bool tail1 = !pair && t >= n4;
        // No divergent branch inside the loop (the LDS reads of q then
        // batch instead of each waiting alone): pair is uniform, and a
        // single-head tail key's odd steps go to c by selects.
        if (pair) {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const float4 q0 = *(const float4*)(qs + 8 * i + 4 * h);
                const float4 q1 = *(const float4*)(qs + HD + 8 * i + 4 * h);
                const float4 kk = kr[i];
                a[0] = fmaf(q0.x, kk.x, a[0]); a[1] = fmaf(q0.y, kk.y, a[1]);
                a[2] = fmaf(q0.z, kk.z, a[2]); a[3] = fmaf(q0.w, kk.w, a[3]);
                b[0] = fmaf(q1.x, kk.x, b[0]); b[1] = fmaf(q1.y, kk.y, b[1]);
                b[2] = fmaf(q1.z, kk.z, b[2]); b[3] = fmaf(q1.w, kk.w, b[3]);
            }
        } else {
#pragma unroll
            for (int i = 0; i < NI; i++) {
                const float4 q0 = *(const float4*)(qs + 8 * i + 4 * h);
                const float4 kk = kr[i];
                const float qv[4] = {q0.x, q0.y, q0.z, q0.w}, kv[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
                for (int jj = 0; jj < 4; jj++) {
                    if (i & 1) {
                        const float x = fmaf(qv[jj], kv[jj], tail1 ? c[jj] : a[jj]);
                        c[jj] = tail1 ? x : c[jj];
                        a[jj] = tail1 ? a[jj] : x;
                    } else {
                        a[jj] = fmaf(qv[jj], kv[jj], a[jj]);
                    }
                }
            }
        }
        float s0, s1 = 0.0f;
        if (t < n4) {
            // hsum4_256_ps: ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)); lane 0 holds a0..a3
            const float l0 = (a[0] + a[1]) + (a[2] + a[3]);
            const float l1 = (b[0] + b[1]) + (b[2] + b[3]);
            const float o0 = fxor1(l0), o1 = fxor1(l1);
            s0 = (h ? o0 + l0 : l0 + o0) * scale;
            s1 = (h ? o1 + l1 : l1 + o1) * scale;
        } else {
            if (tail1) {
#pragma unroll
                for (int jj = 0; jj < 4; jj++) a[jj] = a[jj] + c[jj];
            }
            // eng_hsum256_ps: ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
            float u[4], ub[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const float pa = fxor1(a[jj]), pb = fxor1(b[jj]);
                u[jj] = h ? pa + a[jj] : a[jj] + pa;
                ub[jj] = h ? pb + b[jj] : b[jj] + pb;
            }
            s0 = ((u[0] + u[1]) + (u[2] + u[3])) * scale;
            s1 = ((ub[0] + ub[1]) + (ub[2] + ub[3])) * scale;
        }
        if (t < kv_len) {
            if (h == 0) {
                sc0[t] = s0;
                if (pair) sc1[t] = s1;
            }
        }
    }
    __syncthreads();  // score rows complete
    // Softmax of head w by wave w alone, keys lane + 64 r: the maximum, the
    // exponentials (exp_poly below n8, libm expf for the tail), the
    // reference's 8 sum chains (lane j: keys j, j + 8, ... below n8 in order),
    // hsum8, the tail in order, and the normalisation.  The wave reads back
    // rows it wrote itself (LDS operations of one wave complete in order), so
    // no workgroup barrier falls between the steps.
    const int n8 = kv_len & ~7;
    if (wave < nh) {
        constexpr int KPL = (DPUF_HIP_DEC_MAX_KEYS + 63) / 64;
        float* sp = wave ? sc1 : sc0;
        float ev[KPL];
        float mx = -1e30f;
#pragma unroll
        for (int r = 0; r < KPL; r++) {
            const int t = lane + 64 * r;
            ev[r] = t < kv_len ? sp[t] : -1e30f;
            mx = ev[r] > mx ? ev[r] : mx;
        }
        mx = wave_max(mx);
#pragma unroll
        for (int r = 0; r < KPL; r++) {
            const int t = lane + 64 * r;
            if (t < kv_len) {
                ev[r] = t < n8 ? exp_poly(ev[r] - mx) : expf_libc_tab(ev[r] - mx, etab);
                sp[t] = ev[r];
            }
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's rows are in LDS
        __builtin_amdgcn_wave_barrier();
        float inv = 0.0f;
        if (lane < 8) {
            constexpr int NS = DPUF_HIP_DEC_MAX_KEYS / 8;
            float pv[NS];
#pragma unroll
            for (int i = 0; i < NS; i++) pv[i] = lane + 8 * i < n8 ? sp[lane + 8 * i] : 0.0f;
            float a = 0.0f;
#pragma unroll
            for (int i = 0; i < NS; i++)
                if (lane + 8 * i < n8) a = a + pv[i];
            vs8[wave][lane] = a;
        }
        __builtin_amdgcn_s_waitcnt(0xc07f);
        __builtin_amdgcn_wave_barrier();
        if (lane == 0) {
            float tl[7];  // the tail (at most 7 keys), loaded before its ordered adds
#pragma unroll
            for (int i = 0; i < 7; i++) tl[i] = n8 + i < kv_len ? sp[n8 + i] : 0.0f;
            float su = hsum8(vs8[wave]);
#pragma unroll
            for (int i = 0; i < 7; i++)
                if (n8 + i < kv_len) su += tl[i];
            inv = 1.0f / (su + 1e-12f);
        }
        inv = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(inv)));
#pragma unroll
        for (int r = 0; r < KPL; r++) {
            const int t = lane + 64 * r;
            if (t < kv_len) sp[t] = ev[r] * inv;
        }
    }

    // P.V over LDS chunks of V (row pos comes from vn); output o = (hsel, d)
    constexpr int NO = (2 * HD + 255) / 256;
    float acc[NO];
#pragma unroll
    for (int jo = 0; jo < NO; jo++) acc[jo] = 0.0f;
    for (int c0 = 0; c0 < kv_len; c0 += V_ROWS) {
        if (c0 > 0) {
            __syncthreads();  // previous chunk consumed
            stage_v(c0, kv_len - c0 < V_ROWS ? kv_len - c0 : V_ROWS);
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (pos >= c0 && pos < c0 + V_ROWS) {
            for (int i = tid; i < HD; i += 256) vst[(pos - c0) * HD + i] = vn[i];
            __syncthreads();
        }
        const int cn = kv_len - c0 < V_ROWS ? kv_len - c0 : V_ROWS;
#pragma unroll
        for (int jo = 0; jo < NO; jo++) {
            const int o = tid + 256 * jo;
            if (o >= nh * HD) break;
            const int hsel = o / HD, d = o % HD;
            const float* p = (hsel ? sc1 : sc0) + c0;
            const float* vcol = vst + d;
            float a = acc[jo];
            int r = 0;
            if (pair) {
                for (; r + 8 <= cn; r += 8) {
                    float pv[8], vv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        pv[u] = p[r + u];
                        vv[u] = vcol[(r + u) * HD];
                    }
#pragma unroll
                    for (int u = 0; u < 8; u++) a = fmaf(pv[u], vv[u], a);
                }
                for (; r < cn; r++) a = fmaf(p[r], vcol[r * HD], a);
            } else {
                for (; r + 8 <= cn; r += 8) {
                    float pv[8], vv[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) {
                        pv[u] = p[r + u];
                        vv[u] = vcol[(r + u) * HD];
                    }
#pragma unroll
                    for (int u = 0; u < 8; u += 2) a = fmaf(pv[u], vv[u], fmaf(pv[u + 1], vv[u + 1], a));
                }
                for (; r + 1 < cn; r += 2) a = fmaf(p[r], vcol[r * HD], fmaf(p[r + 1], vcol[(r + 1) * HD], a));
                if (r < cn) a = fmaf(p[r], vcol[r * HD], a);
            }
            acc[jo] = a;
        }
    }
    __syncthreads();
#pragma unroll
    for (int jo = 0; jo < NO; jo++) {
        const int o = tid + 256 * jo;
        if (o < nh * HD) {
            aout[o] = acc[jo];
            ao[(size_t)qh0 * HD + o] = acc[jo];
        }
    }
    __syncthreads();
    // prep of the O input for columns [qh0*HD, (qh0+nh)*HD): a wave per
    // 64-block, a column per lane
#pragma unroll
    for (int k = 0; k < NPB; k++) {
        const int b = wave + 4 * k;
        if (b < nh * HD / 64) {
            float x = aout[64 * b + lane];
            if ((osb >> k) & 1u) x = -x;
            wave_prep64(x, lane, (qh0 * HD) / 64 + b, op.q, op.s, op.m, op.h);
        }
    }
}


extern "C" {

int32_t dpuf_hip_attn_dec(void* s, int32_t M, const float* q, const float* k, const float* v, const float* q_norm,
                          const float* k_norm, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                          float* vc, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                          float scale, float* ao, const uint8_t* o_sign, DpufPrep op, float* const* kcs,
                          float* const* vcs, size_t l_off, DpufWarm warm) {
    if (M < 1) return -1;
    warm.n_wg = 0;
    if (M == 1 && warm.sink && warm.n_jobs > 0) {
        // one warm-up workgroup on every CU the attention leaves idle
        const int n_cu = dpuf_hip_cu_count(), busy = n_kv * ((n_q / n_kv + 1) / 2);
        warm.n_wg = n_cu > busy + 8 ? (n_cu - busy) & ~7 : 0;
    }
    if (M == 1) op.h = NULL;  // the one-row GEMV reads q only
    const int groups = n_q / n_kv;
    const size_t scl = 2 * (size_t)DPUF_HIP_DEC_MAX_KEYS > 3 * (size_t)hd ? 2 * (size_t)DPUF_HIP_DEC_MAX_KEYS
                                                                       : 3 * (size_t)hd;
    const size_t lds = ((size_t)16384 + (size_t)6 * hd + scl) * sizeof(float);
    const dim3 grid(n_kv, (groups + 1) / 2 + (warm.n_wg + n_kv - 1) / n_kv, M);
#define ATT_LAUNCH(HDV)                                                                                            \
    hipLaunchKernelGGL(k_attn_dec<HDV>, grid, dim3(256), lds, ST(s), q, k, v, q_norm, k_norm, eps, cos_tab, sin_tab, \
                       kc, vc, pos0, n_q, n_kv, max_seq, scale, ao, o_sign, op, kcs, vcs, l_off, warm)
    switch (hd) {
        case 64: ATT_LAUNCH(64); break;
        case 128: ATT_LAUNCH(128); break;
        case 256: ATT_LAUNCH(256); break;
        default: return -1;
    }
#undef ATT_LAUNCH
    LAUNCHED("k_attn_dec");
    attn_path_note(4);
    return 0;
}


}  // extern "C"
