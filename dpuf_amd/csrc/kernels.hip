// kernels.hip -- gfx950 (CDNA4, wave64) kernels of the DPUF Mode 12 token loop
// and the thin extern "C" layer that launches them (hip_layer.h).
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

#include <mutex>

#include "hip_layer.h"
#include "dev_common.h"


// ---------------------------------------------------------------------------
// Error bookkeeping
// ---------------------------------------------------------------------------
// First HIP error of the current API call on this thread: every entry point
// of the library clears it on entry (dpuf_hip_clear_error) and reports it on
// exit, so one failed call does not fail the next one or another thread's.
static thread_local hipError_t g_err = hipSuccess;
static thread_local char g_err_msg[256];

static void note(hipError_t e, const char* what) {
    if (e != hipSuccess && g_err == hipSuccess) {
        g_err = e;
        snprintf(g_err_msg, sizeof g_err_msg, "%s: %s", what, hipGetErrorString(e));
    }
}
#define CK(x) note((x), #x)
#define LAUNCHED(name) note(hipGetLastError(), name)

void dpuf_note(hipError_t e, const char* what) { note(e, what); }

// exp for x <= 0 with the results of the host C library's expf, which the
// reference calls on the scalar tail of its softmax (dpuf_engine.c:423-426).
// Method: exp(x) = 2^(k/32) * 2^(r/32), k = round(x*32/ln2), with a 32-entry
// table of 2^(i/32) and a cubic polynomial evaluated in double precision,
// rounded once to float (the exp2f-table method of Szabolcs Nagy used by
// glibc's expf).  The table holds bits(2^(i/32)) - (i << 47), i.e. the
// correctly rounded doubles 2^(i/32) with the exponent contribution removed.
// Checked bit-for-bit against glibc expf over every float in [-104, 0].
__constant__ uint64_t c_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// tab: the 32 table words (c_exp2_tab, or a copy in LDS: a kernel whose
// tail exponentials sit on its critical path copies the table at entry, so
// the lookup does not wait for a global load).
DEV float expf_libc_tab(float x, const uint64_t* tab) {
    if (x < -0x1.9fe368p6f) return 0.0f;  // below log(2^-150): rounds to +0
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    double xd = (double)x;
    double kd = fma(inv_ln2_n, xd, shift);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki & 31u] + (ki << 47);
    double sc = __longlong_as_double((long long)t);
    double z = fma(c0, r, c1);
    double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    y = y * sc;
    return (float)y;
}

DEV float expf_libc(float x) { return expf_libc_tab(x, c_exp2_tab); }

// ---------------------------------------------------------------------------
// Embedding (reference dpuf_embed_qr_hadamard4_packed_f32, dpuf_avx2.c:2738-2783,
// and embed_qr_had_asym_impl, dpuf_avx2.c:3154-3207, for modes 13 / 14)
// grid: M rows; thread per 64-column block.
// ---------------------------------------------------------------------------
// ids (and pos_src) may sit in fine-grained host memory that the host wrote
// just before the launch: system-scope loads read them past every cache.
// Workgroup 0 copies the step's start position to pos_dst in device memory,
// where the kernels after it read it, and the step serial the host put next
// to it (pos_src[1]) to serial_dst.
__global__ void k_embed(DpufDevW w, const int32_t* __restrict__ ids, const float* __restrict__ embeds,
                        float* __restrict__ out, const int32_t* pos_src, int32_t* pos_dst, int32_t* serial_dst) {
    const int m = blockIdx.x;
    const int H = w.cols, n_blk = H >> 5;
    float* dst = out + (size_t)m * H;
    if (pos_dst && m == 0 && threadIdx.x == 0)
        *pos_dst = __hip_atomic_load(pos_src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (serial_dst && m == 0 && threadIdx.x == 0)
        *serial_dst = __hip_atomic_load(pos_src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int id = ids ? __hip_atomic_load(ids + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : -1;
    if (embeds && id < 0) {
        // H is a multiple of 64: float4 copies, eight loads in flight per thread
        const float4* src4 = (const float4*)(embeds + (size_t)m * H);
        float4* dst4 = (float4*)dst;
        const int n4 = H >> 2, T = blockDim.x;
        for (int i0 = threadIdx.x; i0 < n4; i0 += 8 * T) {
            float4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) v[k] = i0 + k * T < n4 ? src4[i0 + k * T] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (i0 + k * T < n4) dst4[i0 + k * T] = v[k];
        }
        return;
    }
    const int g = id >> 3, ri = id & 7;
    const bool asym = w.mode != 12, hi6 = w.mode == 14;
    const uint8_t* grp = w.g + (size_t)g * n_blk * (hi6 ? 208 : 144);
    const uint16_t* sc = (const uint16_t*)grp;
    const uint8_t* qg = grp + (size_t)n_blk * 16;
    for (int blk = threadIdx.x; blk < (H >> 6); blk += blockDim.x) {
        float v[64];
        // modes 13 / 14: (float)u * d + m, a rounded product then a rounded
        // sum (dpuf_avx2.c:3194-3195); mode 12: (u - 8) * ws
        const float wd = h2f(sc[2 * blk * 8 + ri]), wm = h2f(sc[(2 * blk + 1) * 8 + ri]);
#pragma unroll
        for (int hb = 0; hb < 2; hb++) {
            const int b = 2 * blk + hb;
            const float ws = h2f(sc[b * 8 + ri]);
            const uint4 rw = *(const uint4*)(qg + (size_t)b * 128 + ri * 16);
            const uint32_t words[4] = {rw.x, rw.y, rw.z, rw.w};
            uint2 hw = make_uint2(0u, 0u);
            if (hi6) hw = *(const uint2*)(grp + (size_t)n_blk * 144 + ((size_t)b * 8 + ri) * 8);
            const uint32_t hws[2] = {hw.x, hw.y};
#pragma unroll
            for (int c = 0; c < 4; c++) {
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t by = (words[c] >> (8 * k)) & 0xFFu;
                    if (asym) {
                        const uint32_t hb2 = (hws[c >> 1] >> (8 * k + (c & 1) * 4)) & 0xFu;
                        const int u0 = (int)((by & 15u) | ((hb2 & 3u) << 4));
                        const int u1 = (int)((by >> 4) | ((hb2 >> 2) << 4));
                        v[32 * hb + 8 * c + k] = (float)u0 * wd + wm;
                        v[32 * hb + 8 * c + 4 + k] = (float)u1 * wd + wm;
                    } else {
                        v[32 * hb + 8 * c + k] = (float)((int)(by & 15u) - 8) * ws;
                        v[32 * hb + 8 * c + 4 + k] = (float)((int)(by >> 4) - 8) * ws;
                    }
                }
            }
        }
        fwht64(v);
        if (w.sign) {
#pragma unroll
            for (int bb = 0; bb < 8; bb++) {
                const uint32_t sb = w.sign[8 * blk + bb];
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if ((sb >> k) & 1u) v[8 * bb + k] = -v[8 * bb + k];
            }
        }
        float4* d4 = (float4*)(dst + 64 * blk);
#pragma unroll
        for (int i = 0; i < 16; i++) d4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    }
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

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

// ---------------------------------------------------------------------------
// Residual add + RMSNorm + prep for up to three sign vectors (reference
// add_and_rms_norm_f32, dpuf_engine.c:243-272, then the prep above).
// grid: M rows; block: H/16 threads, thread t owning columns 16t..16t+15.
// The sum of squares keeps the reference's 8 FMA lanes (lane j accumulates
// elements j, j+8, j+16, ... in order) and its hsum tree; a transposed LDS
// copy gives each of the 8 chain lanes its elements contiguously.
// ---------------------------------------------------------------------------
//
// G = 4 (H a multiple of 256, no xn_out): four workgroups per row
// (blockIdx.y), each running the whole sum chain and then the prep of a
// quarter of the row's 64-blocks, a block per 16-lane row with 4 columns
// per lane (row_prep64): the prep's per-lane work, which bounds it, is a
// sixteenth of one workgroup doing every block by lane quads.  Every
// workgroup reads h + res, so the sum goes to h_out (not in place); each
// writes its quarter.
template <int SEG, int G>
__global__ __launch_bounds__(1024) void k_resnorm_prep(int H, const float* h, const float* __restrict__ res, float* h_out,
                                                       const float* __restrict__ w,
                                                       float eps, PrepSet ps, float* __restrict__ xn_out) {
    extern __shared__ float tr[];  // [8][H/8 + 4]
    __shared__ float part[8];
    const int m = blockIdx.x, t = threadIdx.x, qp = t & 3, blk = t >> 2, nb = H >> 5;
    const int L = (H >> 3) + 4;
    const int T = H >> 4;  // threads
    float v[16], wv[16];
    uint32_t sb[3];
    // G = 4: block b4 of the row (a quarter's 16-lane rows), lane r4, its
    // 4 columns, their norm weights and sign bits
    const int b4 = (int)blockIdx.y * (H >> 8) + (t >> 4), r4 = t & 15, c4 = 64 * b4 + 4 * r4;
    float4 w4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    load16(h + (size_t)m * H + 16 * t, v);
    if (G == 1) {
        load16(w + 16 * t, wv);
        for (int p = 0; p < 3; p++) sb[p] = p < ps.n ? quad_sign_bits(ps.sign[p], blk, qp) : 0u;
    } else {
        w4 = *(const float4*)(w + c4);
        for (int p = 0; p < 3; p++)
            sb[p] = p < ps.n && ps.sign[p] ? (ps.sign[p][8 * b4 + (r4 >> 1)] >> (4 * (r4 & 1))) & 0xFu : 0u;
    }
    if (res) {
        float r[16];
        load16(res + (size_t)m * H + 16 * t, r);
#pragma unroll
        for (int k = 0; k < 16; k++) v[k] = v[k] + r[k];
        if (G == 1 || (t >> 2) / (T >> 4) == (int)blockIdx.y)  // this workgroup's quarter
            store16(h_out + (size_t)m * H + 16 * t, v);
    }
#pragma unroll
    for (int k = 0; k < 8; k++) *(float2*)(tr + k * L + 2 * t) = make_float2(v[k], v[k + 8]);
    __syncthreads();
    if (SEG > 0) {
        // H = 64 SEG.  Chain j (lanes 8j .. 8j+7 of wave 0) in 8 consecutive
        // segments of SEG elements held in registers: lane 8j + s runs
        // segment s, then hands the accumulator to lane 8j + s + 1 (DPP
        // row_shr:1, inside a 16-lane row).  A register-fed dependent fma
        // costs about 1.9 ns on gfx950 against 4-5 ns fed from LDS; the order
        // is the reference's.
        if (t < 64) {
            const int j = t >> 3, s = t & 7;
            const float4* rowp = (const float4*)(tr + j * L + s * SEG);
            float x[SEG > 0 ? SEG : 1];
#pragma unroll
            for (int i = 0; i < SEG / 4; i++) {
                const float4 e = rowp[i];
                x[4 * i] = e.x;
                x[4 * i + 1] = e.y;
                x[4 * i + 2] = e.z;
                x[4 * i + 3] = e.w;
            }
            float a = 0.0f;
#pragma unroll
            for (int ss = 0; ss < 8; ss++) {
                if (s == ss) {
#pragma unroll
                    for (int i = 0; i < SEG; i++) a = fmaf(x[i], x[i], a);
                }
                const float prev = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x111, 0xF, 0xF,
                                                                              false));
                if (s == ss + 1) a = prev;
            }
            if (s == 7) part[j] = a;
        }
    } else if (t < 8) {
        const float4* row = (const float4*)(tr + t * L);
        const int n4 = H >> 5;
        float a = 0.0f;
        int i = 0;
        for (; i + 4 <= n4; i += 4) {
            const float4 e0 = row[i], e1 = row[i + 1], e2 = row[i + 2], e3 = row[i + 3];
            a = fmaf(e0.x, e0.x, a); a = fmaf(e0.y, e0.y, a); a = fmaf(e0.z, e0.z, a); a = fmaf(e0.w, e0.w, a);
            a = fmaf(e1.x, e1.x, a); a = fmaf(e1.y, e1.y, a); a = fmaf(e1.z, e1.z, a); a = fmaf(e1.w, e1.w, a);
            a = fmaf(e2.x, e2.x, a); a = fmaf(e2.y, e2.y, a); a = fmaf(e2.z, e2.z, a); a = fmaf(e2.w, e2.w, a);
            a = fmaf(e3.x, e3.x, a); a = fmaf(e3.y, e3.y, a); a = fmaf(e3.z, e3.z, a); a = fmaf(e3.w, e3.w, a);
        }
        for (; i < n4; i++) {
            const float4 e = row[i];
            a = fmaf(e.x, e.x, a); a = fmaf(e.y, e.y, a); a = fmaf(e.z, e.z, a); a = fmaf(e.w, e.w, a);
        }
        part[t] = a;
    }
    __syncthreads();
    const float inv = 1.0f / sqrtf(hsum8(part) / (float)H + eps);
    if (G > 1) {
        // element e of the row is tr[(e % 8) L + e / 8]
        const float wk[4] = {w4.x, w4.y, w4.z, w4.w};
        float x0[4];
#pragma unroll
        for (int k = 0; k < 4; k++) x0[k] = (tr[((c4 + k) & 7) * L + ((c4 + k) >> 3)] * inv) * wk[k];
        for (int p = 0; p < ps.n; p++) {
            float y[4];
#pragma unroll
            for (int k = 0; k < 4; k++) y[k] = ((sb[p] >> k) & 1u) ? -x0[k] : x0[k];
            row_prep64(y, r4, b4, ps.p[p].q + (size_t)m * H, ps.p[p].s + (size_t)m * nb, ps.p[p].m + (size_t)m * nb,
                       ps.p[p].h ? ps.p[p].h + (size_t)m * H : nullptr);
        }
        return;
    }
#pragma unroll
    for (int k = 0; k < 16; k++) v[k] = (v[k] * inv) * wv[k];
    if (xn_out) store16(xn_out + (size_t)m * H + 16 * t, v);
    for (int p = 0; p < ps.n; p++) {
        float y[16];
#pragma unroll
        for (int k = 0; k < 16; k++) y[k] = v[k];
        apply_sign_bits(y, sb[p]);
        quad_fwht64(y, qp);
        quad_quant_store(y, qp, blk, ps.p[p].q + (size_t)m * H, ps.p[p].s + (size_t)m * nb, ps.p[p].m + (size_t)m * nb,
                         ps.p[p].h ? ps.p[p].h + (size_t)m * H : nullptr);
    }
}

// Plain activation prep of M rows of x [M][K].  grid: (ceil(K/16/256), M).
__global__ __launch_bounds__(256) void k_prep(int K, const float* __restrict__ x, const uint8_t* __restrict__ sign,
                                              DpufPrep p) {
    const int m = blockIdx.y, t = blockIdx.x * blockDim.x + threadIdx.x;
    if (16 * t >= K) return;  // whole quads: K is a multiple of 64
    const int qp = t & 3, blk = t >> 2, nb = K >> 5;
    float v[16];
    load16(x + (size_t)m * K + 16 * t, v);
    apply_sign_bits(v, quad_sign_bits(sign, blk, qp));
    quad_fwht64(v, qp);
    quad_quant_store(v, qp, blk, p.q + (size_t)m * K, p.s + (size_t)m * nb, p.m + (size_t)m * nb,
                     p.h ? p.h + (size_t)m * K : nullptr);
}

// Lane t of one row: columns 4t .. 4t + 3 of the 64-block t / 16 (COH: see
// row_prep64).
template <bool COH = false>
DEV void swiglu_prep_lane(int I, const float* __restrict__ gate, const float* __restrict__ up, float dz,
                          const uint8_t* __restrict__ sign, int8_t* q, float* s, int32_t* m, uint16_t* h, int t) {
    const int blk = t >> 4, r = t & 15;
    const float4 g4 = *(const float4*)(gate + 4 * t);
    const float4 u4 = *(const float4*)(up + 4 * t);
    const uint32_t sb = sign ? (sign[8 * blk + (r >> 1)] >> (4 * (r & 1))) & 0xFu : 0u;
    const float g[4] = {g4.x, g4.y, g4.z, g4.w}, u[4] = {u4.x, u4.y, u4.z, u4.w};
    float v[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float ng = fmaxf(-40.0f, fminf(0.0f - g[k], 40.0f));
        const float silu = g[k] / (1.0f + exp_poly(ng));
        float rr = silu * u[k];
        if (dz > 0.0f && !(fabsf(rr) >= dz)) rr = 0.0f;
        v[k] = ((sb >> k) & 1u) ? -rr : rr;
    }
    row_prep64<COH>(v, r, blk, q, s, m, h);
}

// The plain prep of lane t of one row (columns 4t .. 4t + 3): sign, then
// row_prep64 (COH: see row_prep64).
template <bool COH = false>
DEV void prep_lane(const float* __restrict__ x, const uint8_t* __restrict__ sign, int8_t* q, float* s, int32_t* m, int t) {
    const int blk = t >> 4, r = t & 15;
    const float4 x4 = *(const float4*)(x + 4 * t);
    const uint32_t sb = sign ? (sign[8 * blk + (r >> 1)] >> (4 * (r & 1))) & 0xFu : 0u;
    float v[4] = {x4.x, x4.y, x4.z, x4.w};
#pragma unroll
    for (int k = 0; k < 4; k++) v[k] = ((sb >> k) & 1u) ? -v[k] : v[k];
    row_prep64<COH>(v, r, blk, q, s, m, nullptr);
}

// SwiGLU with dead zone (reference swiglu_range_avx2, 8-wide path,
// dpuf_engine.c:976-989) fused with the prep of the down projection's input.
// A 64-block per 16-lane row, 4 columns per lane (row_prep64): a quarter of
// the per-lane work of a quad per block, which is what bounds this
// latency-bound step.  grid: (ceil(I / 256), M), one wave per workgroup.
__global__ __launch_bounds__(64) void k_swiglu_prep(int I, const float* __restrict__ gate, const float* __restrict__ up,
                                                    float dz, const uint8_t* __restrict__ sign, DpufPrep p) {
    const int m = blockIdx.y, t = blockIdx.x * 64 + threadIdx.x;
    const int nb = I >> 5;
    if (64 * (t >> 4) >= I) return;  // whole rows: I is a multiple of 64
    swiglu_prep_lane(I, gate + (size_t)m * I, up + (size_t)m * I, dz, sign, p.q + (size_t)m * I, p.s + (size_t)m * nb,
                     p.m + (size_t)m * nb, p.h ? p.h + (size_t)m * I : nullptr, t);
}

// ---------------------------------------------------------------------------
// Mode 12 matrices in HBM: the row-block layout.
//
// A .dpuf group (8 rows) holds [n_blk][8] fp16 scales, then per 32-column
// block b four 32-byte chunks; byte ri*4+k of chunk c holds row ri, column
// 32b+8c+k (low nibble) and 32b+8c+4+k (high nibble) (dpuf_avx2.c:2347-2353).
// At upload k_relayout stores every group densely (group g of a matrix at
// g * n_blk * 144; tile headers and padding dropped) and gathers each row's
// four chunk words of a block into 16 contiguous bytes:
//   row ri, block b: byte b*128 + ri*16 + 4c + k  <-  .dpuf b*128 + c*32 + ri*4 + k
// One 16-byte load then gives a lane a whole 32-column row block, and the 64
// lanes of a wave (lane = 8*bi + ri) read 8 blocks x 8 rows = 1 KB with
// consecutive addresses.  Scales stay [n_blk][8]: lane (bi, ri) of step s
// reads scale s*64 + lane.
// ---------------------------------------------------------------------------
//
// Modes 13 / 14 (asymmetric blk64, dpuf_avx2.c:2786-2791) have the same group
// prefix: their [n_64][16] fp16 (d of rows 0..7, then m) is, viewed as
// [n_blk][8], "block" 2j = d and 2j+1 = m of 64-block j, and their nibbles
// use the mode 12 interleave, so the same gather applies (144 bytes per 32
// columns).  Mode 14 then holds per block 64 bytes of bits 4..5: bits
// 2(ri>>1) of byte c*16 + h*8 + (ri&1)*4 + k belong to row ri, column
// 32b+8c+4h+k.  Those are regathered per row into two words, word w byte k =
// chunk 2w's columns +k, +4+k in bits 0-1, 2-3 and chunk 2w+1's in bits 4-5,
// 6-7, stored after the nibbles: row ri, block b at n_blk*144 + (b*8+ri)*8.
// ---------------------------------------------------------------------------
__global__ void k_relayout(const uint8_t* __restrict__ src, const uint64_t* __restrict__ offs, int n_groups,
                           int n_blk, int hi6, uint8_t* __restrict__ dst) {
    const size_t total = (size_t)n_groups * n_blk * 8;
    const size_t gbytes = (size_t)n_blk * (hi6 ? 208 : 144);
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int g = (int)(idx / ((size_t)n_blk * 8));
        const int rem = (int)(idx % ((size_t)n_blk * 8));
        const int b = rem >> 3, ri = rem & 7;
        const uint8_t* sg = src + offs[g >> 1] + 16 + (size_t)(g & 1) * gbytes;
        uint8_t* dg = dst + (size_t)g * gbytes;
        ((uint16_t*)dg)[b * 8 + ri] = ((const uint16_t*)sg)[b * 8 + ri];
        const uint32_t* sq = (const uint32_t*)(sg + (size_t)n_blk * 16 + (size_t)b * 128);
        *(uint4*)(dg + (size_t)n_blk * 16 + (size_t)b * 128 + ri * 16) =
            make_uint4(sq[ri], sq[8 + ri], sq[16 + ri], sq[24 + ri]);
        if (hi6) {
            const uint8_t* sh = sg + (size_t)n_blk * 144 + (size_t)b * 64 + (ri & 1) * 4;
            const int sft = (ri >> 1) * 2;
            uint32_t w[2] = {0u, 0u};
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int h = 0; h < 2; h++)
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        const uint32_t hv = (sh[c * 16 + h * 8 + k] >> sft) & 3u;
                        w[c >> 1] |= hv << (8 * k + (c & 1) * 4 + h * 2);
                    }
            *(uint2*)(dg + (size_t)n_blk * 144 + ((size_t)b * 8 + ri) * 8) = make_uint2(w[0], w[1]);
        }
    }
}

// The same for a mode 14 row block: bits 4..5 of each value come from the
// row's two words of high bits (word c >> 1, bits (c & 1) * 4 + {0,1} of byte
// k for column 8c+k, + {2,3} for 8c+4+k).  u <= 63, so the sdot4 products are
// exact, as the reference's maddubs sums (dpuf_avx2.c:2824-2846).
DEV int row_block_dot6(uint4 w, uint2 hw, int4 xa, int4 xb) {
    const uint32_t m = 0x0F0F0F0Fu, m2 = 0x03030303u;
    const uint32_t wd[4] = {w.x, w.y, w.z, w.w};
    const int xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    int d = 0;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t h = ((c >> 1) ? hw.y : hw.x) >> ((c & 1) * 4);
        const uint32_t lo = (wd[c] & m) | ((h & m2) << 4);
        const uint32_t hi = ((wd[c] >> 4) & m) | (((h >> 2) & m2) << 4);
        d = __builtin_amdgcn_sdot4((int)lo, xw[2 * c], d, false);
        d = __builtin_amdgcn_sdot4((int)hi, xw[2 * c + 1], d, false);
    }
    return d;
}

// Per-row fp32 chain acc = fma(float(D - sum8), ws * xs, acc) over blocks in
// ascending order (dpuf_avx2.c:2633-2635); `row` holds (dcf, sp) pairs, two
// per float4, n_blk even.  Pairs are read in batches of NB float4 with the
// next batch in flight while the current one is consumed, so LDS latency
// stays off the dependent FMA chain (about 13 cycles per FMA on gfx950).
template <int NB>
DEV void chain_batch(const float4* e, float& acc) {
#pragma unroll
    for (int i = 0; i < NB; i++) {
        acc = fmaf(e[i].x, e[i].y, acc);
        acc = fmaf(e[i].z, e[i].w, acc);
    }
}

template <int NB>
DEV float run_chain(const float4* row, int n2) {
    float acc = 0.0f;
    int k = 0;
    if (n2 >= 2 * NB) {
        float4 cur[NB], nxt[NB];
#pragma unroll
        for (int i = 0; i < NB; i++) cur[i] = row[i];
        for (k = NB; k + NB <= n2; k += NB) {
#pragma unroll
            for (int i = 0; i < NB; i++) nxt[i] = row[k + i];
            chain_batch<NB>(cur, acc);
#pragma unroll
            for (int i = 0; i < NB; i++) cur[i] = nxt[i];
        }
        chain_batch<NB>(cur, acc);
    }
    for (; k < n2; k++) {
        const float4 e = row[k];
        acc = fmaf(e.x, e.y, acc);
        acc = fmaf(e.z, e.w, acc);
    }
    return acc;
}

// ---------------------------------------------------------------------------
// M == 1 GEMV.
//
// A step is 8 blocks x 8 rows of one 8-row group = 1 KB of nibbles, one
// 16-byte load per lane (lane = 8*bi + ri: row ri of block 8s + bi), plus the
// lane's fp16 scale.  A workgroup has NW loader waves, each taking NL
// consecutive steps of a group per round (R rounds per group).  The fp32
// chains of a group, acc = fma(float(D - sum8), ws * xs, acc) over its blocks
// in ascending order (dpuf_avx2.c:2633-2635), are one dependent FMA per block
// (about 13 cycles each on gfx950), so how they are scheduled decides the
// kernel's speed.  Two launch modes:
//
// One group per workgroup (SINGLE), when the chip holds a workgroup for every
// group at once: load, dots to LDS, one barrier, lanes 0..7 of wave 0 chain.
//
// Persistent workgroups, when there are more groups: job j gets
// wb[j+1] - wb[j] workgroups, sized so the whole grid is resident, and
// workgroup lb of the job walks the job's groups lb, lb + nwg, ...  With one
// round per group (every K up to 14336) a loader wave always works on the
// same steps, so its 32 activation bytes, scale and sum per step are loaded
// into registers once and the steady state issues only the weight and scale
// loads, one (group, round) unit ahead.  Dots go to LDS as
// (float(D - sum8), ws * xs) pairs [row][block] in one of up to MV_NBUF
// rotating buffers; after its last round of a group a loader wave counts
// itself in with an LDS atomic and goes on without waiting.  MV_NC extra
// chain waves take the groups in turn (group lg -> chain wave lg % MV_NC),
// wait for the group's loader waves, run its 8 row chains on lanes 0..7 and
// free the buffer, so chains overlap the loads of later groups; a loader
// wave only waits when it is MV_NBUF groups ahead of the chains.
//
// In both modes blocks whose activation scale is <= 0 contribute nothing, as
// the M == 1 reference skips them (dpuf_avx2.c:2621-2622): their pair is
// (0, 0), which leaves a chain unchanged (an accumulator is never -0).
// ---------------------------------------------------------------------------
#define MV_NBUF 4   // pair buffers in flight per workgroup
#define MV_CHAIN 4  // float4 pairs per LDS read batch of a chain (chain waves)
#define MV_CHAIN1 8  // the same for the one-group-per-workgroup instances
#define MV_NC 2     // chain waves per workgroup
// Launch-shape choice (compile-time): whether groups of 43..56 steps (K up to
// 14336) keep their activations in registers (11..14 loader waves x 4 steps)
// or load them per round.
#define MV_HOIST48 1

struct MvJob {
    const uint8_t* g;  // dense groups of the matrix (row-block layout)
    float* out;        // row r of the matrix -> out[r]
    int g0, g1;        // groups computed by this launch
    int rows;
    DpufPrep x;        // prepped activations (row 0)
};

struct MvArgs {
    MvJob j[3];
    int n_jobs;
    int wb[4];  // prefix sums of the workgroups given to each job
    int K;
    int nbuf;   // pair buffers in LDS: min(MV_NBUF, most groups of one workgroup)
    int nc;     // chain waves: MV_NC, or 0 when every workgroup has one group
    const int32_t* skip_flag;
    float fill;
    int32_t* err;  // device error word: bit 0 set when a bounded LDS wait ran out
    // Producer-fed launch (one job, one group per workgroup, activations
    // held for the launch): the first np workgroups compute the job's
    // activations, SwiGLU + dead zone + prep of gate pg / up pu [pI]
    // (k_swiglu_prep's arithmetic), or with pu NULL the plain prep of pg
    // (k_prep's), and each sets its flag pflag[p] to the step serial *pep;
    // the GEMV workgroups after them issue their weight loads first and read
    // the activations once every flag holds the serial.
    int np, pI;
    const float* pg;
    const float* pu;
    float pdz;
    const uint8_t* psign;
    int32_t* pflag;
    const int32_t* pep;
};

// Activations of one round of one wave.
template <int NL>
struct MvX {
    int4 xa[NL], xb[NL];
    float xs[NL];
    int32_t xm[NL];
};

// Loads of one unit (a round of one group) of one wave; x only when the
// activations are not held for the whole launch.
template <int NL>
struct MvU {
    uint4 wq[NL];
    uint2 wh[NL];  // mode 14: the row block's bits 4..5
    uint32_t ws[NL];
    MvX<NL> x;
};

// Uniform over the workgroup.
struct MvGeo {
    int n_blk, S, ld, R, NW;
    int lb, nwg;     // this workgroup's index within its job, the job's workgroup count
    int nbuf;        // pair buffers in LDS (<= MV_NBUF)
    const uint8_t* g;
    float* out;
    int g0, rows;
    DpufPrep x;
    int32_t* err;
};

// A bounded wait that ran out leaves its buffer's data incomplete: the launch
// goes on (every wave still ends) and the host, which reads this word after
// the call, reports the call as failed.
DEV void mv_wait_failed(int32_t* err) { atomicOr(err, 1); }

// Waits until *p == want, at most 2^22 polls; false when it ran out.  The
// polled value is made wave-uniform, so the loop is a scalar loop: a
// per-lane loop condition made the compiler unroll the waits eightfold with
// an exec mask per step, doubling the kernel's SGPRs (one wave per SIMD
// fewer) and its code.
template <typename T>
DEV bool mv_wait(T* p, T want) {
    int spins = 0;
#pragma clang loop unroll(disable)
    while ((T)__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) !=
           want) {
        if (++spins >= (1 << 22)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

// Loads are unconditional (indices clamped into the group), so the number of
// memory operations in flight is the same on every path and the wait for one
// unit never includes the next unit's loads.
template <int NL>
DEV void mv_load_x(const MvGeo& G, int r, int w, int lane, MvX<NL>& X) {
    const int s0 = (r * G.NW + w) * NL;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int s = min(s0 + i, G.S - 1);
        const uint32_t b = (uint32_t)min(s * 8 + (lane >> 3), G.n_blk - 1);
        X.xa[i] = *(const int4*)(G.x.q + b * 32u);
        X.xb[i] = *(const int4*)(G.x.q + b * 32u + 16u);
        X.xs[i] = G.x.s[b];
        X.xm[i] = G.x.m[b];
    }
}

template <int NL, bool HOIST, int MODE>
DEV void mv_issue(const MvGeo& G, int u, int w, int lane, MvU<NL>& L) {
    const int lg = u / G.R, r = u - lg * G.R;
    const int g = G.g0 + G.lb + lg * G.nwg;
    const uint8_t* grp = G.g + (size_t)g * G.n_blk * (MODE == 14 ? 208 : 144);
    const uint16_t* sc = (const uint16_t*)grp;
    const uint8_t* qg = grp + (size_t)G.n_blk * 16;
    const uint8_t* hg = grp + (size_t)G.n_blk * 144;
    const int s0 = (r * G.NW + w) * NL;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int s = min(s0 + i, G.S - 1);
        const uint32_t b = (uint32_t)min(s * 8 + (lane >> 3), G.n_blk - 1);
        const uint32_t e = b * 8u + (uint32_t)(lane & 7);  // == 64 s + lane unless clamped
        L.wq[i] = nt_load16(qg + e * 16u);
        if (MODE == 14) L.wh[i] = *(const uint2*)(hg + e * 8u);
        L.ws[i] = sc[e];
    }
    if (!HOIST) mv_load_x<NL>(G, r, w, lane, L.x);
}

// Mode 12: (float(D - sum8), ws * xs) pairs of one round of one wave into
// pairs[row][block].  Modes 13 / 14: the two 32-blocks 2j, 2j+1 of 64-block
// j sit on lanes (bi, ri) and (bi + 1, ri), 8 lanes apart, and swap their dot,
// activation scale and sum over DPP; the even lane writes (fdot, d) with
// fdot = fma(float(D0), xs0, float(D1) * xs1), the odd lane (m, xm_s) with
// xm_s = ((float)sum8_0 * xs0 + (float)sum8_1 * xs1) * 0.125f, so the chain
// fma(a, b, acc) over the pairs in order is the reference's
// acc = fma(fdot, d, acc); acc = fma(m, xm_s, acc) (dpuf_avx2.c:3029-3037).
template <int NL, bool HOIST, int MODE>
DEV void mv_dots(const MvGeo& G, int r, int w, int lane, const MvU<NL>& L, const MvX<NL>& X0, float2* pairs) {
    const MvX<NL>& X = HOIST ? X0 : L.x;
    const int bi = lane >> 3, ri = lane & 7;
    const int s0 = (r * G.NW + w) * NL;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        const int s = s0 + i;
        if (s >= G.S) break;  // wave-uniform
        const int b = s * 8 + bi;
        if (MODE != 12) {
            const int dot = MODE == 14 ? row_block_dot6(L.wq[i], L.wh[i], X.xa[i], X.xb[i])
                                       : row_block_dot(L.wq[i], X.xa[i], X.xb[i]);
            const int dp = dpp_ror8(dot), xmp = dpp_ror8(X.xm[i]);
            const float xsp = __int_as_float(dpp_ror8(__float_as_int(X.xs[i])));
            const float sc = h2f((uint16_t)L.ws[i]);
            float2 pr;
            if ((bi & 1) == 0) {
                pr.x = fmaf((float)dot, X.xs[i], (float)dp * xsp);
                pr.y = sc;
            } else {
                const float a = (float)xmp * xsp, c = (float)X.xm[i] * X.xs[i];
                pr.x = sc;
                pr.y = (a + c) * 0.125f;
            }
            if (b < G.n_blk) pairs[ri * G.ld + b] = pr;
            continue;
        }
        if (b < G.n_blk) {
            const int dot = row_block_dot(L.wq[i], X.xa[i], X.xb[i]);
            float dcf = 0.0f, sp = 0.0f;
            if (X.xs[i] > 0.0f) {
                dcf = (float)(dot - X.xm[i]);
                sp = h2f((uint16_t)L.ws[i]) * X.xs[i];
            }
            pairs[ri * G.ld + b] = make_float2(dcf, sp);
        }
    }
}

// LDS bookkeeping of the pair buffers: loader-wave arrivals per buffer
// (cumulative over the launch) and the last group whose chains finished in it.
struct MvSync {
    uint32_t cnt[MV_NBUF];
    int32_t done[MV_NBUF];
};

template <int NL, bool HOIST, int MODE>
DEV void mv_consume(const MvGeo& G, int u, int w, int lane, const MvU<NL>& L, const MvX<NL>& X0, uint8_t* smem,
                    MvSync* sy) {
    const int lg = u / G.R, r = u - lg * G.R;
    const int buf = lg % G.nbuf;
    float2* pairs = (float2*)smem + (size_t)buf * 8 * G.ld;
    if (r == 0 && lg >= G.nbuf) {
        // the buffer is free once the chains of group lg - nbuf have read it
        if (!mv_wait(&sy->done[buf], (int32_t)(lg - G.nbuf)) && lane == 0) mv_wait_failed(G.err);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    mv_dots<NL, HOIST, MODE>(G, r, w, lane, L, X0, pairs);
    if (r == G.R - 1) {
        // publish this wave's pairs of the group to the chain wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_fetch_add(&sy->cnt[buf], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// The chain wave: for each group of the workgroup in order, wait until all
// loader waves have published their pairs, run the 8 rows' chains on lanes
// 0..7 at raised issue priority, write the rows, free the buffer.  Every wait
// is bounded.
DEV void mv_chains(const MvGeo& G, int c, int n_my, int lane, uint8_t* smem, MvSync* sy) {
    for (int lg = c; lg < n_my; lg += MV_NC) {
        const int buf = lg % G.nbuf;
        // arrivals in this buffer are cumulative: use lg / nbuf of the buffer is
        // complete at NW * (lg / nbuf + 1), and the next use cannot start
        // arriving before this group's chains free the buffer
        const uint32_t want = (uint32_t)G.NW * (uint32_t)(lg / G.nbuf + 1);
        if (!mv_wait(&sy->cnt[buf], want) && lane == 0) mv_wait_failed(G.err);
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        __builtin_amdgcn_s_setprio(2);
        if (lane < 8) {
            const float2* pairs = (const float2*)smem + (size_t)buf * 8 * G.ld;
            const float acc = run_chain<MV_CHAIN>((const float4*)(pairs + lane * G.ld), G.n_blk >> 1);
            const int r = (G.g0 + G.lb + lg * G.nwg) * 8 + lane;
            if (r < G.rows) G.out[r] = acc;
        }
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_store(&sy->done[buf], lg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// Flags of a producer-fed launch: MV_FLAG_COPIES copies of the np flags, 64
// apart; a GEMV workgroup polls the copy of its XCD (workgroup b runs on XCD
// b % 8), so the polls of the launch spread over that many cache lines.
#define MV_FLAG_COPIES 8

// Producer workgroup p of a producer-fed launch: lanes p * blockDim .. of
// the SwiGLU + prep row, written with agent-scope stores (past the L2, to
// where every XCD reads: no L2 writeback, which walks the whole cache).
// Every wave waits until its stores are done; after the barrier the flag
// copies take the step serial.
DEV void mv_produce(const MvArgs& A, int p) {
    const int t = p * (int)blockDim.x + (int)threadIdx.x;
    const DpufPrep& P = A.j[0].x;
    if (64 * (t >> 4) < A.pI) {
        if (A.pu) swiglu_prep_lane<true>(A.pI, A.pg, A.pu, A.pdz, A.psign, P.q, P.s, P.m, nullptr, t);
        else prep_lane<true>(A.pg, A.psign, P.q, P.s, P.m, t);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const int32_t ep = *A.pep;
        for (int c = 0; c < MV_FLAG_COPIES; c++)
            __hip_atomic_store(A.pflag + 64 * c + p, ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Until every producer flag holds ep (lane i polls flag i, agent-scope
// loads, which see the producers' written-back stores); at most 2^20 polls,
// false when they ran out.  The exit test is a ballot: wave-uniform.
DEV bool mv_wait_producers(const int32_t* flags, int np, int32_t ep, int lane) {
    int spins = 0;
#pragma clang loop unroll(disable)
    while (true) {
        const int32_t f = lane < np ? __hip_atomic_load(flags + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ep;
        if (__ballot(f != ep) == 0) return true;
        if (++spins >= (1 << 20)) return false;
        __builtin_amdgcn_s_sleep(2);
    }
}

// FED: the producer-fed mode (one group per workgroup, activations held),
// an instance of its own so the other instances keep their registers.
template <int NL, bool HOIST, bool SINGLE, int MODE, bool FED = false>
__global__ __launch_bounds__(1024) void k_mv(MvArgs A) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    int bid = blockIdx.x;
    if (FED) {
        if (bid < A.np) {
            mv_produce(A, bid);
            return;
        }
        bid -= A.np;
    }
    int ji = 0;
    if (A.n_jobs > 1 && bid >= A.wb[1]) ji = 1;
    if (A.n_jobs > 2 && bid >= A.wb[2]) ji = 2;
    const MvJob& J = A.j[ji];
    MvGeo G;
    G.lb = bid - A.wb[ji];
    G.nwg = A.wb[ji + 1] - A.wb[ji];
    G.g = J.g;
    G.out = J.out;
    G.g0 = J.g0;
    G.rows = J.rows;
    G.x = J.x;
    G.err = A.err;
    const int n_my = (J.g1 - J.g0 - G.lb + G.nwg - 1) / G.nwg;
    if (A.skip_flag && *A.skip_flag) {
        for (int lg = 0; lg < n_my; lg++) {
            const int r0 = (G.g0 + G.lb + lg * G.nwg) * 8;
            if (tid < 8 && r0 + tid < G.rows) G.out[r0 + tid] = A.fill;
        }
        return;
    }
    G.NW = (blockDim.x >> 6) - A.nc;  // loader waves; the last A.nc waves run the chains
    G.n_blk = A.K >> 5;
    G.S = (G.n_blk + 7) >> 3;
    G.ld = G.n_blk + 2;
    G.R = HOIST ? 1 : (G.S + G.NW * NL - 1) / (G.NW * NL);
    const int n_units = n_my * G.R;
    G.nbuf = A.nbuf;
    __shared__ MvSync sy;
    if (tid < MV_NBUF) {
        sy.cnt[tid] = 0u;
        sy.done[tid] = -1;
    }
    __syncthreads();
    if (w >= G.NW) {
        mv_chains(G, w - G.NW, n_my, lane, smem, &sy);
        return;
    }
    if (SINGLE) {
        // one group per workgroup: no chain waves, one barrier, wave 0 chains
        MvX<NL> X1;
        MvU<NL> L1;
        if (FED) {
            // producer-fed (one round: HOIST): the weights first, then this
            // step's producer flags, then the activations they published
            const int32_t ep = *A.pep;
            mv_issue<NL, HOIST, MODE>(G, 0, w, lane, L1);
            // one wave polls (the flag lines see one load per workgroup and
            // poll, not one per wave); the others wait at the barrier
            if (w == 0 && !mv_wait_producers(A.pflag + 64 * (blockIdx.x % MV_FLAG_COPIES), A.np, ep, lane) &&
                lane == 0)
                mv_wait_failed(G.err);
            __syncthreads();
            // Plain loads see the producers' data: every cache level was
            // invalidated when the launch began and no wave of it touches
            // these lines before their flags are set (only the flags, which
            // change during the launch, need the agent-scope polls).
            __atomic_signal_fence(__ATOMIC_SEQ_CST);  // the activation loads stay after the wait
            mv_load_x<NL>(G, 0, w, lane, X1);
            mv_dots<NL, HOIST, MODE>(G, 0, w, lane, L1, X1, (float2*)smem);
        } else {
            if (HOIST) mv_load_x<NL>(G, 0, w, lane, X1);
            for (int r = 0; r < G.R; r++) {
                mv_issue<NL, HOIST, MODE>(G, r, w, lane, L1);
                mv_dots<NL, HOIST, MODE>(G, r, w, lane, L1, X1, (float2*)smem);
            }
        }
        __syncthreads();
        if (w == 0 && lane < 8) {
            const float acc = run_chain<MV_CHAIN1>((const float4*)((float2*)smem + lane * G.ld), G.n_blk >> 1);
            const int r = G.g0 * 8 + G.lb * 8 + lane;
            if (r < G.rows) G.out[r] = acc;
        }
        return;
    }
    MvX<NL> X;
    if (HOIST) mv_load_x<NL>(G, 0, w, lane, X);
    // Steady state: both issues unconditional, so each consume waits only for
    // its own loads; the last one or two units drain after the loop.
    MvU<NL> La, Lb;
    mv_issue<NL, HOIST, MODE>(G, 0, w, lane, La);
    int u = 0;
    for (; u + 2 < n_units; u += 2) {
        mv_issue<NL, HOIST, MODE>(G, u + 1, w, lane, Lb);
        mv_consume<NL, HOIST, MODE>(G, u, w, lane, La, X, smem, &sy);
        mv_issue<NL, HOIST, MODE>(G, u + 2, w, lane, La);
        mv_consume<NL, HOIST, MODE>(G, u + 1, w, lane, Lb, X, smem, &sy);
    }
    if (u + 1 < n_units) {
        mv_issue<NL, HOIST, MODE>(G, u + 1, w, lane, Lb);
        mv_consume<NL, HOIST, MODE>(G, u, w, lane, La, X, smem, &sy);
        mv_consume<NL, HOIST, MODE>(G, u + 1, w, lane, Lb, X, smem, &sy);
    } else {
        mv_consume<NL, HOIST, MODE>(G, u, w, lane, La, X, smem, &sy);
    }
}

// ---------------------------------------------------------------------------
// M > 1 GEMM on the matrix cores (slab path, dpuf_avx2.c:2643-2676).
//
// For every (row, token) the reference accumulates every block:
//   acc = fma(float(D - sum8), fp16(ws) * xs, acc), blocks ascending,
// with D the u4 x i8 dot of the block and sum8 = 8 * sum(q).  Since
// D - sum8 = sum((u - 8) * q) exactly, one v_mfma_f32_16x16x32_f16 per block
// with A = (u - 8) and B = q, both exact in f16, gives float(D - sum8) for a
// 16-row x 16-token tile (every partial sum is an integer below 2^15, exact
// in the fp32 accumulator).  The epilogue is the reference's two rounded
// operations, sp = ws * xs and the fma, with the chains in registers across
// the block loop, so the block order is the reference's.
//
// A workgroup of 4 waves computes 64 GM_RF rows x 16 TT tokens; wave w owns
// GM_RF 16-row fragments and all the tokens as TT 16-token tiles (GM_RF TT
// MFMAs per block).  Activations arrive as fp16 (DpufPrep.h, written by the
// prep kernels) and are staged in LDS, GM_SB blocks per stage, double-
// buffered, one barrier per stage; a token's 64 bytes per block are four
// 16-byte chunks stored XOR-swizzled by token so a fragment read is free of
// bank conflicts.  A block's fragments are read from LDS one block ahead of
// its MFMAs.  Weights, nibbles and scales, are read straight into registers
// one stage ahead.  MFMA lane layouts (gfx950, checked on the device): A lane
// l = row l % 16, k = 8 (l / 16) + e; B lane l = token l % 16, same k; D lane
// l = token l % 16, rows 4 (l / 16) + v.
// ---------------------------------------------------------------------------
#define GM_SB 4  // blocks per LDS stage
#define GM_RF 1  // 16-row fragments per wave (workgroup = 64 GM_RF rows)
#define GM_TT 4  // 16-token tiles per workgroup
#define GM_XCD 1  // XCD-grouped workgroup order

typedef _Float16 gm_h8 __attribute__((ext_vector_type(8)));
typedef float gm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t gm_u4 __attribute__((ext_vector_type(4)));
#define GM_RSRC3 0x00020000  // buffer descriptor word 3 (gfx9 family): 32-bit raw data

struct GmJob {
    const uint8_t* g;  // dense groups of the matrix
    int g0, g1;        // groups computed
    int rows;
    const uint16_t* h;  // activations as fp16 [M][K]
    const float* s;     // block scales [M][K/32]
    const int32_t* m;   // 8 * block sums of q [M][K/32] (modes 13 / 14)
    float* out;        // out[m * ldo + row]
    int ldo;
};

struct GmArgs {
    GmJob j[3];
    int n_jobs;
    int tb[4];  // prefix sums of 16-group row tiles per job
    int K, M;
    int gy;     // token tiles
    // rows [z0, z1) of zo (row stride zld) set to 0 by zt extra row tiles of
    // 64 rows placed after the jobs' tiles
    float* zo;
    int zld, z0, z1, zt;
};


// A fragment from one nibble word (row i, columns 8 kc .. 8 kc + 7 of a
// block: low nibbles = columns +0..+3, high nibbles = +4..+7): u - 8 as f16.
DEV gm_h8 gm_unpack_a(uint32_t w) {
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    const uint32_t r0 = gm_sub(gm_pair(lo, 0x04010400u), (_Float16)1032.0f);
    const uint32_t r1 = gm_sub(gm_pair(lo, 0x04030402u), (_Float16)1032.0f);
    const uint32_t r2 = gm_sub(gm_pair(hi, 0x04010400u), (_Float16)1032.0f);
    const uint32_t r3 = gm_sub(gm_pair(hi, 0x04030402u), (_Float16)1032.0f);
    return __builtin_bit_cast(gm_h8, make_uint4(r0, r1, r2, r3));
}

// The same for modes 13 / 14: u itself (no offset) as f16, with bits 4..5
// from h (bits 0-1 of byte k for the low half, 2-3 for the high half; 0 for
// mode 13).
DEV gm_h8 gm_unpack_a_asym(uint32_t w, uint32_t h) {
    const uint32_t lo = (w & 0x0F0F0F0Fu) | ((h & 0x03030303u) << 4);
    const uint32_t hi = ((w >> 4) & 0x0F0F0F0Fu) | (((h >> 2) & 0x03030303u) << 4);
    const uint32_t r0 = gm_sub(gm_pair(lo, 0x04010400u), (_Float16)1024.0f);
    const uint32_t r1 = gm_sub(gm_pair(lo, 0x04030402u), (_Float16)1024.0f);
    const uint32_t r2 = gm_sub(gm_pair(hi, 0x04010400u), (_Float16)1024.0f);
    const uint32_t r3 = gm_sub(gm_pair(hi, 0x04030402u), (_Float16)1024.0f);
    return __builtin_bit_cast(gm_h8, make_uint4(r0, r1, r2, r3));
}


// Modes 13 / 14 hold a 64-block's even half (its D tiles, token scales and
// sums, row scales) across the odd one: 2 waves per SIMD keep that in
// registers instead of spilling at the 128 VGPRs of 4.
template <int TT, int RF, int MODE>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(MODE == 12 ? 4 : 2))) void k_gemm_mfma(
    GmArgs A) {
    constexpr int NT = 16 * TT;  // tokens per workgroup
    constexpr bool ASYM = MODE != 12;
    static_assert(GM_SB % 2 == 0, "a stage holds whole 64-blocks");
    __shared__ __align__(16) uint8_t bq[2][GM_SB][NT][64];  // f16 activations [stage][block][token][k]
    __shared__ __align__(16) float bs[2][GM_SB][16][TT];    // block scales [stage][block][token % 16][token / 16]
    __shared__ __align__(16) int32_t bm[ASYM ? 2 : 1][GM_SB][16][TT];  // 8 * block sums (modes 13 / 14)
    __shared__ __align__(16) uint32_t bw[2][GM_SB][32 * RF];  // weight scales [stage][block][group * 4 + word]
    // Workgroups go to the 8 XCDs round-robin by linear id L.  L = xcd +
    // 8 j with j = gy r + ty puts row tile 8 r + xcd of every token tile ty on
    // one XCD, dispatched back to back, so the gy workgroups that read the
    // same weights run together and share them through that XCD's L2.
#if GM_XCD
    const int jx = blockIdx.x >> 3, ty = jx % A.gy;
    const int rt = (jx / A.gy) * 8 + (blockIdx.x & 7);
#else
    const int rt = blockIdx.x, ty = blockIdx.y;
#endif
    if (rt >= A.tb[A.n_jobs]) {
        // zeroing tiles, then padding of the grid (whole workgroups)
        const int zi = rt - A.tb[A.n_jobs];
        if (zi < A.zt) {
            const int r = A.z0 + 64 * zi + (threadIdx.x & 63);
            for (int t = threadIdx.x >> 6; t < 16 * TT; t += 4) {
                const int m = ty * 16 * TT + t;
                if (m < A.M && r < A.z1) A.zo[(size_t)m * A.zld + r] = 0.0f;
            }
        }
        return;
    }
    int ji = 0;
    if (A.n_jobs > 1 && rt >= A.tb[1]) ji = 1;
    if (A.n_jobs > 2 && rt >= A.tb[2]) ji = 2;
    // the job's fields picked from the kernel arguments by uniform selects,
    // so they stay in scalar registers through the loop
    const GmJob& J = ji == 0 ? A.j[0] : ji == 1 ? A.j[1] : A.j[2];
    const uint16_t* const Jh = ji == 0 ? A.j[0].h : ji == 1 ? A.j[1].h : A.j[2].h;
    const float* const Js = ji == 0 ? A.j[0].s : ji == 1 ? A.j[1].s : A.j[2].s;
    const int32_t* const Jm = ji == 0 ? A.j[0].m : ji == 1 ? A.j[1].m : A.j[2].m;
    const int gb = J.g0 + (rt - A.tb[ji]) * 8 * RF;  // first group of the workgroup
    const int m0 = ty * NT;
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, i16 = l & 15, kc = l >> 4;
    const int K = A.K, M = A.M, n_blk = K >> 5;
    const size_t gstride = (size_t)n_blk * (MODE == 14 ? 208 : 144);

    // Every load is a buffer load: a wave-uniform descriptor, a 32-bit lane
    // offset fixed for the launch and a scalar block offset, so addressing
    // costs no vector instructions in the loop (and a load past a
    // descriptor's range reads 0 instead of faulting).  Weights of the
    // wave's RF fragments (groups clamped into the job) are addressed from
    // the wave's first group.
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int gw0 = min(gb + 2 * RF * wu, J.g1 - 1);
    const size_t wbytes = (size_t)(J.g1 - gw0) * gstride;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(J.g + (size_t)gw0 * gstride), 0, (int)(wbytes < 0xFFFFFFFFu ? wbytes : 0xFFFFFFFFu), GM_RSRC3);
    uint32_t on[RF], oh[RF];
#pragma unroll
    for (int f = 0; f < RF; f++) {
        const int ga = min(gb + 2 * RF * wu + 2 * f + (i16 >> 3), J.g1 - 1);
        on[f] = (uint32_t)((size_t)(ga - gw0) * gstride + (size_t)n_blk * 16 + (i16 & 7) * 16 + kc * 4);
        // mode 14: the lane's high-bit word (chunk kc's bits are in word kc / 2)
        oh[f] = (uint32_t)((size_t)(ga - gw0) * gstride + (size_t)n_blk * 144 + (i16 & 7) * 8 + (kc >> 1) * 4);
    }
    // Weight scales go through LDS with the activations: a stage's 8 RF
    // groups x GM_SB blocks x 8 fp16 scales are WD dwords, dword d = (tid +
    // 256 k) % WD (group d / (4 GM_SB), block (d / 4) % GM_SB, word d % 4),
    // addressed from the workgroup's first group; threads past WD repeat a
    // dword.  Blocks past the end read bytes that are never used.
    constexpr int WD = 32 * RF * GM_SB, WPT = (WD + 255) / 256;
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(J.g + (size_t)gb * gstride), 0,
        (int)((size_t)(J.g1 - gb) * gstride < 0xFFFFFFFFu ? (size_t)(J.g1 - gb) * gstride : 0xFFFFFFFFu), GM_RSRC3);
    uint32_t og[WPT], sw[WPT];  // load offsets; the thread's scale dwords of the stage in flight
    int wgi[WPT];               // their LDS word index in a stage buffer
#pragma unroll
    for (int k = 0; k < WPT; k++) {
        const int wd = (tid + 256 * k) % WD, g = wd / (4 * GM_SB), b = (wd >> 2) % GM_SB, w4 = wd & 3;
        og[k] = (uint32_t)((size_t)(min(gb + g, J.g1 - 1) - gb) * gstride + b * 16 + w4 * 4);
        wgi[k] = b * 32 * RF + g * 4 + w4;
    }
    // staging: a stage holds NT tokens x GM_SB blocks of 64 fp16 bytes, four
    // 16-byte chunks each.  Chunk c = tid + 256 k of the stage is chunk c & 3
    // of pair c / 4 = (token (c / 4) % NT, block (c / 4) / NT), so the 64
    // lanes of a load read 16 tokens' 64 contiguous bytes.  Scale i = tid +
    // 256 k is pair i.  Loads are unconditional, at token and block clamped
    // into range: a token past M only feeds output columns that are never
    // stored, a block past the end is never computed, and a load without a
    // branch around it keeps the compiler's wait counts exact.
    constexpr int CPT = NT * GM_SB * 4 / 256, SPT = (NT * GM_SB + 255) / 256;
    static_assert(CPT >= 1 && NT * GM_SB * 4 % 256 == 0, "whole chunks per thread");
    const int n_st = (n_blk + GM_SB - 1) / GM_SB;
    gm_u4 sq[CPT];  // a native vector: a struct copy would keep the array in scratch
    float ss[SPT];
    int32_t sm[SPT];
    // byte offsets of the token rows (M K < 2^30 is checked at launch); with
    // NT = 64 a chunk's block (k) and a scale's block (the wave, + 4 k) are
    // uniform and go into the scalar offset
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)Jh, 0, M * K * 2, GM_RSRC3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)Js, 0, M * n_blk * 4, GM_RSRC3);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc(ASYM ? (void*)Jm : (void*)Js, 0, M * n_blk * 4, GM_RSRC3);
    uint32_t ho[CPT], so[SPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int pr = (tid >> 2) + 64 * k, m = min(m0 + pr % NT, M - 1);
        const int sbt = NT == 64 ? 0 : pr / NT;
        ho[k] = (uint32_t)(2 * (m * K + 32 * sbt + 8 * (tid & 3)));
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int i = min(tid + 256 * k, NT * GM_SB - 1), m = min(m0 + i % NT, M - 1);
        const int sbt = NT == 64 ? 0 : i / NT;
        so[k] = (uint32_t)(4 * (m * n_blk + sbt));
    }
    // the stage's first block, clamped so that a stage's blocks stay in range
    // when it starts in range (blocks past the end are never computed)
    auto stage_load = [&](int st) {
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int sbt = NT == 64 ? k : 0;
            const int b = NT == 64 ? min(st * GM_SB + sbt, n_blk - 1) : st * GM_SB;
            sq[k] = __builtin_bit_cast(gm_u4, __builtin_amdgcn_raw_buffer_load_b128(rh, ho[k], b * 64, 0));
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int b = NT == 64 ? min(st * GM_SB + wu + 4 * k, n_blk - 1) : st * GM_SB;
            ss[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, so[k], b * 4, 0));
            if (ASYM) sm[k] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rm, so[k], b * 4, 0);
        }
#pragma unroll
        for (int k = 0; k < WPT; k++) sw[k] = __builtin_amdgcn_raw_buffer_load_b32(rg, og[k], st * GM_SB * 16, 0);
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = tid + 256 * k, pr = c >> 2, tk = pr % NT, sbt = pr / NT, qu = c & 3;
            *(gm_u4*)&bq[buf][sbt][tk][16 * (qu ^ ((tk >> 1) & 3))] = sq[k];
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int i = tid + 256 * k, tk = i % NT, sbt = i / NT;
            if (NT * GM_SB % 256 == 0 || i < NT * GM_SB) {
                bs[buf][sbt][tk & 15][tk >> 4] = ss[k];
                if (ASYM) bm[ASYM ? buf : 0][sbt][tk & 15][tk >> 4] = sm[k];
            }
        }
#pragma unroll
        for (int k = 0; k < WPT; k++) (&bw[buf][0][0])[wgi[k]] = sw[k];
    };
    // nibble words (and mode 14 high-bit words) of one stage, per fragment and block
    uint32_t wn[2][GM_SB][RF];
    uint32_t wh[2][GM_SB][RF];
    auto weights_load = [&](int st, uint32_t (&n)[GM_SB][RF], uint32_t (&hn)[GM_SB][RF]) {
#pragma unroll
        for (int sb = 0; sb < GM_SB; sb++) {
            const int b = min(st * GM_SB + sb, n_blk - 1);
#pragma unroll
            for (int f = 0; f < RF; f++) {
                n[sb][f] = __builtin_amdgcn_raw_buffer_load_b32(rw, on[f], b * 128, 0);
                hn[sb][f] = MODE == 14 ? __builtin_amdgcn_raw_buffer_load_b32(rw, oh[f], b * 64, 0) : 0u;
            }
        }
    };

    gm_f4 acc[RF][TT];
#pragma unroll
    for (int f = 0; f < RF; f++)
#pragma unroll
        for (int t = 0; t < TT; t++) acc[f][t] = (gm_f4){0.0f, 0.0f, 0.0f, 0.0f};

    // B fragments, token scales and the lane's 4 row scales of one block,
    // read from LDS one block ahead of its MFMAs so the read latency hides
    // behind the block before.  The row scales stay two separate 32-bit
    // words: this compiler selected the first word's register for both
    // words' fp16 halves when they came as one 2 x 32-bit vector into
    // v_fma_mix_f32.
    gm_h8 bfr[2][TT];
    float xsr[2][TT];
    int32_t xmr[2][TT];
    uint32_t wsr[2][RF][2];
    auto lds_b = [&](int buf, int sb, int slot) {
#pragma unroll
        for (int f = 0; f < RF; f++) {
            const int e = (2 * (RF * wu + f) + (kc >> 1)) * 4 + (kc & 1) * 2;
            wsr[slot][f][0] = bw[buf][sb][e];
            wsr[slot][f][1] = bw[buf][sb][e + 1];
        }
#pragma unroll
        for (int t = 0; t < TT; t++) xsr[slot][t] = bs[buf][sb][i16][t];
        if (ASYM) {
#pragma unroll
            for (int t = 0; t < TT; t++) xmr[slot][t] = bm[ASYM ? buf : 0][sb][i16][t];
        }
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const int tok = 16 * t + i16;
            bfr[slot][t] = *(const gm_h8*)&bq[buf][sb][tok][16 * (kc ^ ((tok >> 1) & 3))];
        }
    };
    // modes 13 / 14: the even block of a 64-block pair waits in registers for
    // the odd one: its D tiles, token scales and sums, and the lane's 4 d
    gm_f4 dk[RF][TT];
    float xs0k[TT];
    int32_t xm0k[TT];
    float dsk[RF][4];
    auto compute = [&](int st, int buf, const uint32_t (&n)[GM_SB][RF], const uint32_t (&hn)[GM_SB][RF]) {
        lds_b(buf, 0, 0);
#pragma unroll
        for (int sb = 0; sb < GM_SB; sb++) {
            if (st * GM_SB + sb >= n_blk) break;  // uniform
            if (sb + 1 < GM_SB) lds_b(buf, sb + 1, (sb + 1) & 1);
            __builtin_amdgcn_sched_barrier(0);
            gm_h8 a[RF];
            _Float16 wsh[RF][4];
#pragma unroll
            for (int f = 0; f < RF; f++) {
                a[f] = ASYM ? gm_unpack_a_asym(n[sb][f], (hn[sb][f] >> ((kc & 1) * 4)))
                            : gm_unpack_a(n[sb][f]);
                const gm_h2 lo = __builtin_bit_cast(gm_h2, wsr[sb & 1][f][0]),
                            hi = __builtin_bit_cast(gm_h2, wsr[sb & 1][f][1]);
                wsh[f][0] = lo[0];
                wsh[f][1] = lo[1];
                wsh[f][2] = hi[0];
                wsh[f][3] = hi[1];
            }
            float xs[TT];
#pragma unroll
            for (int t = 0; t < TT; t++) xs[t] = xsr[sb & 1][t];
            if (ASYM) {
                // 64-block epilogue (dpuf_avx2.c:2871-2882), rows 4 kc' + v
                // of the fragment for token 16 t + i16:
                //   fdot = fma(float(D0), xs0, float(D1) * xs1)
                //   acc = fma(fdot, d, acc); acc = fma(m, xm_s, acc)
                if ((sb & 1) == 0) {
#pragma unroll
                    for (int t = 0; t < TT; t++) {
                        xs0k[t] = xs[t];
                        xm0k[t] = xmr[sb & 1][t];
#pragma unroll
                        for (int f = 0; f < RF; f++)
                            dk[f][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[f], bfr[sb & 1][t],
                                                                              (gm_f4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                    }
#pragma unroll
                    for (int f = 0; f < RF; f++)
#pragma unroll
                        for (int v = 0; v < 4; v++) dsk[f][v] = (float)wsh[f][v];
                } else {
#pragma unroll
                    for (int t = 0; t < TT; t++) {
                        const float pa = (float)xm0k[t] * xs0k[t], pb = (float)xmr[sb & 1][t] * xs[t];
                        const float xms = (pa + pb) * 0.125f;
#pragma unroll
                        for (int f = 0; f < RF; f++) {
                            const gm_f4 d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                a[f], bfr[sb & 1][t], (gm_f4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; v++) {
                                const float p1 = d1[v] * xs[t];
                                const float fd = fmaf(dk[f][t][v], xs0k[t], p1);
                                acc[f][t][v] = fmaf(fd, dsk[f][v], acc[f][t][v]);
                                acc[f][t][v] = fmaf((float)wsh[f][v], xms, acc[f][t][v]);
                            }
                        }
                    }
                }
                continue;
            }
#pragma unroll
            for (int t = 0; t < TT; t++) {
                const gm_h8 bf = bfr[sb & 1][t];
#pragma unroll
                for (int f = 0; f < RF; f++) {
                    // float(ws) * xs as one mixed-precision FMA with a +0
                    // addend: the same rounding as the product, and a zero
                    // product's sign cannot reach acc, which is never -0.
                    // All four before their uses, so no product is read by
                    // the instruction right after the one writing it.
                    float wx[4];
#pragma unroll
                    for (int v = 0; v < 4; v++) wx[v] = __builtin_fmaf((float)wsh[f][v], xs[t], 0.0f);
                    const gm_f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[f], bf, (gm_f4){0.0f, 0.0f, 0.0f, 0.0f},
                                                                         0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) acc[f][t][v] = fmaf(d[v], wx[v], acc[f][t][v]);
                }
            }
        }
    };

    // prologue: stage 0 into LDS buffer 0, weights of stage 0
    stage_load(0);
    weights_load(0, wn[0], wh[0]);
    stage_store(0);
    __syncthreads();
    int st = 0;
    for (; st + 2 <= n_st; st += 2) {
        stage_load(st + 1);
        weights_load(st + 1, wn[1], wh[1]);
        compute(st, 0, wn[0], wh[0]);
        stage_store(1);
        __syncthreads();
        // on the last pair this stages clamped data that is never computed;
        // the loop body has no branch around its loads
        stage_load(st + 2);
        weights_load(st + 2, wn[0], wh[0]);
        compute(st + 1, 1, wn[1], wh[1]);
        stage_store(0);
        __syncthreads();
    }
    if (st < n_st) compute(st, 0, wn[0], wh[0]);

    // rows 16 RF w + 16f + 4kc + v of the workgroup, token m0 + 16t + i16
#pragma unroll
    for (int f = 0; f < RF; f++) {
        const int grp = gb + 2 * RF * w + 2 * f + (kc >> 1);
        if (grp >= J.g1) continue;
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const int m = m0 + 16 * t + i16;
            if (m >= M) continue;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int r = grp * 8 + (kc & 1) * 4 + v;
                if (r < J.rows) J.out[(size_t)m * J.ldo + r] = acc[f][t][v];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// M <= 16 GEMM (one 16-token tile): the chains of k_gemm_mfma with K split
// across the waves of a workgroup.
//
// With one token tile k_gemm_mfma has one wave per 16 rows, each streaming
// all of K: a 4096-row matrix keeps only 256 waves busy.  Here a workgroup
// computes one 16-row fragment (2 groups) for the M tokens.  SK_NP producer
// waves take the blocks of a round (SKP_RB consecutive blocks each, SKP_RS
// per round): one v_mfma_f32_16x16x32_f16 per block gives float(D - sum8) of
// the 16 x 16 tile exactly, stored to LDS.  SK_NC = 4 chain waves run the
// fp32 chains one round behind: chain wave c owns output (token l % 16, row
// 4 (l / 16) + c) of the MFMA D layout and applies the round's blocks in
// ascending order, acc = fma(d, fp16(ws) * xs, acc), the same two rounded
// operations as k_gemm_mfma, so every output is bit-identical to it.  One
// barrier per round hands the (double-buffered) D tiles over.
//
// A producer wave reads its 4 blocks with one 16-byte load per lane (lane
// (row i, kc): row i's 16 bytes of block b0 + kc) and a 4 x 4 lane transpose
// restores the MFMA A layout (skp_transpose).  Weights, scales and
// activations are loaded SK_P - 1 rounds ahead into a register ring, the
// round loop unrolled by SK_P so every slot index is static: all in one ring
// because the wait counter retires loads in issue order, so activations
// loaded later than the weights would hold every wait to the newest weights.
// The scales ride in the same ring: 32 lanes of each producer wave load the
// weight-scale dwords of the wave's blocks and store them transposed,
// [row][block], so a chain lane reads its row's scales of a round with 16-byte
// LDS reads, and every lane a token scale, [token][block]; the chains read
// LDS only, so no memory latency sits between two barriers.
// ---------------------------------------------------------------------------
#define SK_NP 8   // producer waves
#define SK_NC 4   // chain waves (one per D component)
#define SK_P 4    // load ring depth in rounds (even; fastest of 4..10 in a sweep of the dword-load version)
static_assert(SK_P % 2 == 0, "the D buffers alternate with the round");

#define SKP_P 8  // ring depth in rounds: a multiple of every NR
#define SKP_RB 4                 // blocks per producer wave per round
#define SKP_RS (SK_NP * SKP_RB)  // 32 blocks per round

// 4 x 4 transpose of (16-lane row, register): afterwards register j of lane
// row g holds what register g of lane row j held.
DEV void skp_transpose(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    // rows 2, 3 of r0 <-> rows 0, 1 of r2; the same for r1, r3
    const auto a = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    // rows 1, 3 of the first <-> rows 0, 2 of the second
    const auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    const auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    r0 = c[0];
    r1 = c[1];
    r2 = d[0];
    r3 = d[1];
}

__global__ __launch_bounds__(64 * (SK_NP + SK_NC)) void k_gemm_sk(GmArgs A) {
    __shared__ __align__(16) float dq[2][SKP_RS][4][64];    // D tiles [buf][block][v][lane]
    __shared__ __align__(16) uint16_t wsl[2][16][SKP_RS];   // weight scales [buf][row][block]
    __shared__ __align__(16) float xsl[2][16][SKP_RS + 4];  // token scales [buf][token][block], rows padded
    const int fr = blockIdx.x;
    // the wave index through readfirstlane: uniform for the compiler, so the
    // role branch and every scalar block offset stay scalar
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
    const int M = A.M;
    if (fr >= A.tb[A.n_jobs]) {
        const int zi = fr - A.tb[A.n_jobs];
        if (zi < A.zt) {
            const int r = A.z0 + 64 * zi + l;
            for (int t = w; t < M; t += SK_NP + SK_NC)
                if (r < A.z1) A.zo[(size_t)t * A.zld + r] = 0.0f;
        }
        return;
    }
    int ji = 0;
    if (A.n_jobs > 1 && fr >= A.tb[1]) ji = 1;
    if (A.n_jobs > 2 && fr >= A.tb[2]) ji = 2;
    const GmJob& J = ji == 0 ? A.j[0] : ji == 1 ? A.j[1] : A.j[2];
    const uint16_t* const Jh = ji == 0 ? A.j[0].h : ji == 1 ? A.j[1].h : A.j[2].h;
    const float* const Js = ji == 0 ? A.j[0].s : ji == 1 ? A.j[1].s : A.j[2].s;
    const int gf = J.g0 + 2 * (fr - A.tb[ji]);  // first group of the fragment
    const int K = A.K, n_blk = K >> 5, n_r = (n_blk + SKP_RS - 1) / SKP_RS;
    const size_t gstride = (size_t)n_blk * 144;
    const int i16 = l & 15, kc = l >> 4;

    if (w < SK_NP) {
        // ---- producer: 4 blocks per round, one 16-byte weight load per lane
        // (row i16, block b0 + kc) and the lane transpose, as in k_gemm_skp;
        // groups and blocks clamped per lane ----
        const size_t wbytes = (size_t)(J.g1 - gf) * gstride;
        const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(J.g + (size_t)gf * gstride), 0, (int)(wbytes < 0xFFFFFFFFu ? wbytes : 0xFFFFFFFFu), GM_RSRC3);
        const int ga = min(gf + (i16 >> 3), J.g1 - 1);
        const uint32_t on = (uint32_t)((size_t)(ga - gf) * gstride + (size_t)n_blk * 16 + (i16 & 7) * 16);
        const int sj = (l >> 2) & 3, sd = l & 3, sg = min(gf + ((l >> 4) & 1), J.g1 - 1);
        const uint32_t os = (uint32_t)((size_t)(sg - gf) * gstride + sd * 4);
        const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)Jh, 0, M * K * 2, GM_RSRC3);
        const uint32_t ho = (uint32_t)(2 * (min(i16, M - 1) * K + 8 * kc));
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)Js, 0, M * n_blk * 4, GM_RSRC3);
        const int xt = min(i16, M - 1) * n_blk;
        uint32_t wq[SK_P][4], wsq[SK_P];
        gm_u4 ax[SK_P][SKP_RB];
        float xsq[SK_P];
        // weights, scales and activations of round r in one ring slot (the
        // wait counter retires loads in issue order)
        auto load = [&](int r, uint32_t (&q)[4], uint32_t& sq, gm_u4 (&a)[SKP_RB], float& x) {
            const int b0 = r * SKP_RS + w * SKP_RB;
            const gm_u4 v = __builtin_bit_cast(
                gm_u4, __builtin_amdgcn_raw_buffer_load_b128(rw, on + (uint32_t)min(b0 + kc, n_blk - 1) * 128u, 0, 0));
            q[0] = v[0];
            q[1] = v[1];
            q[2] = v[2];
            q[3] = v[3];
            sq = __builtin_amdgcn_raw_buffer_load_b32(rw, os + (uint32_t)min(b0 + sj, n_blk - 1) * 16u, 0, 0);
#pragma unroll
            for (int j = 0; j < SKP_RB; j++)
                a[j] = __builtin_bit_cast(gm_u4,
                                          __builtin_amdgcn_raw_buffer_load_b128(rh, ho, min(b0 + j, n_blk - 1) * 64, 0));
            x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rs, (uint32_t)(4 * (xt + min(b0 + kc, n_blk - 1))), 0, 0));
        };
#pragma unroll
        for (int u = 0; u < SK_P - 1; u++) load(u, wq[u], wsq[u], ax[u], xsq[u]);
        for (int it0 = 0; it0 <= n_r; it0 += SK_P) {
#pragma unroll
            for (int u = 0; u < SK_P; u++) {
                const int it = it0 + u;
                if (it > n_r) break;  // uniform
                const int un = (u + SK_P - 1) % SK_P;
                load(it + SK_P - 1, wq[un], wsq[un], ax[un], xsq[un]);
                if (it < n_r) {
                    const int buf = u & 1;
                    uint32_t t0 = wq[u][0], t1 = wq[u][1], t2 = wq[u][2], t3 = wq[u][3];
                    skp_transpose(t0, t1, t2, t3);
                    const uint32_t tw[4] = {t0, t1, t2, t3};
#pragma unroll
                    for (int j = 0; j < SKP_RB; j++) {
                        const gm_f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            gm_unpack_a(tw[j]), __builtin_bit_cast(gm_h8, ax[u][j]),
                            (gm_f4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) dq[buf][w * SKP_RB + j][v][l] = d[v];
                    }
                    if (l < 32) {
                        const int row = ((l >> 4) & 1) * 8 + 2 * sd;
                        wsl[buf][row][w * SKP_RB + sj] = (uint16_t)(wsq[u] & 0xFFFFu);
                        wsl[buf][row + 1][w * SKP_RB + sj] = (uint16_t)(wsq[u] >> 16);
                    }
                    xsl[buf][i16][w * SKP_RB + kc] = xsq[u];
                }
                __syncthreads();
            }
        }
        return;
    }

    // ---- chain wave c: output (token l % 16, row 4 (l / 16) + c) ----
    const int c = w - SK_NP, rr = 4 * kc + c;
    float acc = 0.0f;
    for (int it = 0; it <= n_r; it++) {
        if (it >= 1) {
            const int buf = (it + 1) & 1, b0 = (it - 1) * SKP_RS;
            const int nj = min(SKP_RS, n_blk - b0);  // uniform
            float d[SKP_RS];
#pragma unroll
            for (int j = 0; j < SKP_RS; j++) d[j] = dq[buf][j][c][l];
            // scale words as separate 32-bit values (see k_gemm_skp)
            uint32_t wv[SKP_RS / 2];
#pragma unroll
            for (int q = 0; q < SKP_RS / 8; q++) {
                const gm_u4 t = *(const gm_u4*)&wsl[buf][rr][8 * q];
                wv[4 * q] = t[0];
                wv[4 * q + 1] = t[1];
                wv[4 * q + 2] = t[2];
                wv[4 * q + 3] = t[3];
            }
            gm_f4 xr[SKP_RS / 4];
#pragma unroll
            for (int q = 0; q < SKP_RS / 4; q++) xr[q] = *(const gm_f4*)&xsl[buf][i16][4 * q];
#pragma unroll
            for (int j = 0; j < SKP_RS; j++) {
                const gm_h2 hw = __builtin_bit_cast(gm_h2, wv[j >> 1]);
                const float wx = __builtin_fmaf((float)hw[j & 1], xr[j >> 2][j & 3], 0.0f);
                if (j < nj) acc = fmaf(d[j], wx, acc);
            }
        }
        __syncthreads();
    }
    const int grp = gf + (rr >> 3);
    const int r = grp * 8 + (rr & 7);
    if (i16 < M && grp < J.g1 && r < J.rows) J.out[(size_t)i16 * J.ldo + r] = acc;
}

// The same for K <= 32 NR blocks (NR rounds of 32 blocks per fragment, NR
// <= 4), with persistent workgroups: job j gets tb[j + 1] - tb[j]
// workgroups, sized to the chip, and workgroup lb walks the job's fragments
// lb, lb + nwg, ... with one load ring running across fragment boundaries,
// so the ring fills once per workgroup instead of once per fragment.  The
// activations and token scales a producer wave needs are the same for every
// fragment: they are loaded once, before the loop, and the ring holds only
// weight nibbles and weight scales, SKP_P - 1 rounds ahead.  Rounds past the
// matrix's last (K < 1024 NR) compute nothing.
//
// A producer wave takes 4 consecutive blocks per round with one 16-byte load
// per lane: lane (row i, kc) reads row i's 16 bytes of block b0 + kc, 1 KB
// per load instruction (four times the bytes of a dword per lane, for the
// same number of load instructions in flight).  A 4 x 4 transpose across the
// four 16-lane rows of the wave (v_permlane32_swap, then v_permlane16_swap)
// turns that into the MFMA A layout: word kc of each of the 4 blocks in lane
// (i, kc).
// ---------------------------------------------------------------------------
template <int NR>
__global__ __launch_bounds__(64 * (SK_NP + SK_NC)) void k_gemm_skp(GmArgs A) {
    static_assert(SKP_P % NR == 0 && NR <= 4, "ring depth must be a multiple of the rounds per fragment");
    __shared__ __align__(16) float dq[2][SKP_RS][4][64];    // D tiles [buf][block][v][lane]
    __shared__ __align__(16) uint16_t wsl[2][16][SKP_RS];   // weight scales [buf][row][block]
    __shared__ __align__(16) float xsl[2][16][SKP_RS + 4];  // token scales [buf][token][block], rows padded
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63;
    const int M = A.M, bid = blockIdx.x;
    if (bid >= A.tb[A.n_jobs]) {
        const int zi = bid - A.tb[A.n_jobs];
        if (zi < A.zt) {
            const int r = A.z0 + 64 * zi + l;
            for (int t = w; t < M; t += SK_NP + SK_NC)
                if (r < A.z1) A.zo[(size_t)t * A.zld + r] = 0.0f;
        }
        return;
    }
    int ji = 0;
    if (A.n_jobs > 1 && bid >= A.tb[1]) ji = 1;
    if (A.n_jobs > 2 && bid >= A.tb[2]) ji = 2;
    const GmJob& J = ji == 0 ? A.j[0] : ji == 1 ? A.j[1] : A.j[2];
    const uint16_t* const Jh = ji == 0 ? A.j[0].h : ji == 1 ? A.j[1].h : A.j[2].h;
    const float* const Js = ji == 0 ? A.j[0].s : ji == 1 ? A.j[1].s : A.j[2].s;
    const int lb = bid - A.tb[ji], nwg = A.tb[ji + 1] - A.tb[ji];
    const int nf = (J.g1 - J.g0 + 1) >> 1;              // fragments of the job
    const int n_my = (nf - lb + nwg - 1) / nwg;         // >= 1: nwg <= nf
    const int K = A.K, n_blk = K >> 5, S = n_my * NR;   // steps: NR rounds per fragment
    const uint32_t gstride = (uint32_t)n_blk * 144u;    // J.g1 gstride < 2^32 is checked at launch
    const int i16 = l & 15, kc = l >> 4;

    if (w < SK_NP) {
        // ---- producer: one descriptor over the job's groups up to g1; the
        // fragment's base goes into the scalar offset, which the range check
        // does not cover, so the lanes of a fragment's second group add it
        // only when it exists (a one-group fragment re-reads its first), and
        // block indices are clamped per lane ----
        const __amdgpu_buffer_rsrc_t rw =
            __builtin_amdgcn_make_buffer_rsrc((void*)J.g, 0, (int)((uint32_t)J.g1 * gstride), GM_RSRC3);
        const uint32_t on = (uint32_t)n_blk * 16u + (i16 & 7) * 16;
        const bool on_hi = i16 >= 8;
        // weight-scale dword of lane l < 32: group (l >> 4) & 1 of the
        // fragment, block (l >> 2) & 3 of the wave, rows 2 (l & 3), 2 (l & 3) + 1
        const int sj = (l >> 2) & 3, sd = l & 3;
        const bool os_hi = ((l >> 4) & 1) != 0;
        uint32_t wq[SKP_P][4], wsq[SKP_P];
        gm_u4 ax[NR][SKP_RB];
        float xh[NR];  // token l & 15, block l >> 4 of the wave, per round
        {
            const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)Jh, 0, M * K * 2, GM_RSRC3);
            const __amdgpu_buffer_rsrc_t rs =
                __builtin_amdgcn_make_buffer_rsrc((void*)Js, 0, M * n_blk * 4, GM_RSRC3);
            const uint32_t ho = (uint32_t)(2 * (min(i16, M - 1) * K + 8 * kc));
            const int xt = min(i16, M - 1) * n_blk;
#pragma unroll
            for (int r = 0; r < NR; r++) {
                const int b0 = r * SKP_RS + w * SKP_RB;
#pragma unroll
                for (int j = 0; j < SKP_RB; j++)
                    ax[r][j] = __builtin_bit_cast(
                        gm_u4, __builtin_amdgcn_raw_buffer_load_b128(rh, ho, min(b0 + j, n_blk - 1) * 64, 0));
                const uint32_t xo = (uint32_t)(4 * (xt + min(b0 + kc, n_blk - 1)));
                xh[r] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, xo, 0, 0));
            }
        }
        // loads of step s = NR fl + r: fragment lb + fl nwg, round r.  Steps
        // past the workgroup's last fragment re-read that fragment.
        const int fr_last = lb + (n_my - 1) * nwg;
        auto wload = [&](int fl, int r, uint32_t (&q)[4], uint32_t& sq) {
            const int fr = min(lb + fl * nwg, fr_last);
            const uint32_t gb = (uint32_t)(J.g0 + 2 * fr) * gstride;
            const uint32_t g2 = J.g0 + 2 * fr + 1 < J.g1 ? gstride : 0u;  // uniform
            const int b0 = r * SKP_RS + w * SKP_RB;
            const uint32_t von = on + (on_hi ? g2 : 0u) + (uint32_t)min(b0 + kc, n_blk - 1) * 128u;
            const gm_u4 v = __builtin_bit_cast(gm_u4, __builtin_amdgcn_raw_buffer_load_b128(rw, von, gb, 0));
            q[0] = v[0];
            q[1] = v[1];
            q[2] = v[2];
            q[3] = v[3];
            const uint32_t vos = (os_hi ? g2 : 0u) + (uint32_t)min(b0 + sj, n_blk - 1) * 16u + sd * 4;
            sq = __builtin_amdgcn_raw_buffer_load_b32(rw, vos, gb, 0);
        };
#pragma unroll
        for (int u = 0; u < SKP_P - 1; u++) wload(u / NR, u % NR, wq[u], wsq[u]);
        for (int it0 = 0; it0 <= S; it0 += SKP_P) {
#pragma unroll
            for (int u = 0; u < SKP_P; u++) {
                const int it = it0 + u;
                if (it > S) break;  // uniform
                const int un = (u + SKP_P - 1) % SKP_P;
                wload((it0 + u + SKP_P - 1) / NR, un % NR, wq[un], wsq[un]);
                const int r = u % NR;
                if (it < S && r * SKP_RS < n_blk) {
                    const int buf = u & 1;
                    uint32_t t0 = wq[u][0], t1 = wq[u][1], t2 = wq[u][2], t3 = wq[u][3];
                    skp_transpose(t0, t1, t2, t3);
                    const uint32_t tw[4] = {t0, t1, t2, t3};
#pragma unroll
                    for (int j = 0; j < SKP_RB; j++) {
                        const gm_f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            gm_unpack_a(tw[j]), __builtin_bit_cast(gm_h8, ax[r][j]),
                            (gm_f4){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) dq[buf][w * SKP_RB + j][v][l] = d[v];
                    }
                    if (l < 32) {
                        const int row = ((l >> 4) & 1) * 8 + 2 * sd;
                        wsl[buf][row][w * SKP_RB + sj] = (uint16_t)(wsq[u] & 0xFFFFu);
                        wsl[buf][row + 1][w * SKP_RB + sj] = (uint16_t)(wsq[u] >> 16);
                    }
                    xsl[buf][i16][w * SKP_RB + kc] = xh[r];
                }
                __syncthreads();
            }
        }
        return;
    }

    // ---- chain wave c: output (token l % 16, row 4 (l / 16) + c) ----
    const int c = w - SK_NP, rr = 4 * kc + c;
    float acc = 0.0f;
    for (int it0 = 0; it0 <= S; it0 += SKP_P) {
#pragma unroll
        for (int u = 0; u < SKP_P; u++) {
            const int it = it0 + u;
            if (it > S) break;  // uniform
            if (it >= 1) {
                // step it - 1: round r of local fragment fl
                const int um = (u + SKP_P - 1) % SKP_P, r = um % NR;
                const int fl = (u >= 1 ? it0 : it0 - SKP_P) / NR + um / NR;
                const int buf = (u + 1) & 1, b0 = r * SKP_RS;
                const int nj = min(SKP_RS, n_blk - b0);  // uniform, <= 0 past the last round
                if (nj > 0) {
                    float d[SKP_RS];
#pragma unroll
                    for (int j = 0; j < SKP_RS; j++) d[j] = dq[buf][j][c][l];
                    // the scale words as separate 32-bit values: this compiler
                    // selected the wrong register for words 1..3 when they
                    // went from a 4 x 32-bit vector into v_fma_mix_f32
                    uint32_t wv[SKP_RS / 2];
#pragma unroll
                    for (int q = 0; q < SKP_RS / 8; q++) {
                        const gm_u4 t = *(const gm_u4*)&wsl[buf][rr][8 * q];
                        wv[4 * q] = t[0];
                        wv[4 * q + 1] = t[1];
                        wv[4 * q + 2] = t[2];
                        wv[4 * q + 3] = t[3];
                    }
                    gm_f4 xr[SKP_RS / 4];
#pragma unroll
                    for (int q = 0; q < SKP_RS / 4; q++) xr[q] = *(const gm_f4*)&xsl[buf][i16][4 * q];
#pragma unroll
                    for (int j = 0; j < SKP_RS; j++) {
                        const gm_h2 hw = __builtin_bit_cast(gm_h2, wv[j >> 1]);
                        const float wx = __builtin_fmaf((float)hw[j & 1], xr[j >> 2][j & 3], 0.0f);
                        if (j < nj) acc = fmaf(d[j], wx, acc);
                    }
                }
                if (r == NR - 1) {
                    const int fr = lb + fl * nwg;
                    const int grp = J.g0 + 2 * fr + (rr >> 3);
                    const int row = grp * 8 + (rr & 7);
                    if (fr < nf && i16 < M && grp < J.g1 && row < J.rows) J.out[(size_t)i16 * J.ldo + row] = acc;
                    acc = 0.0f;
                }
            }
            __syncthreads();
        }
    }
}

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
// ---------------------------------------------------------------------------
#define AS_KC 64  // keys per scores workgroup

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

// k_attn_sc1: the scores of a one-token step (M = 1) for an even group of at
// most GM query heads.  k_attn_sc's tiling gives each thread two rows and four
// keys, so with G <= 8 rows only G / 2 x 16 threads of a workgroup compute;
// here every thread works: thread (key kq = tid / 4, jp = tid % 4) runs the
// reference's accumulators j = 2 jp and 2 jp + 1 (a[j] = fma chain over i of
// q[8i + j] * k[8i + j]) for all the group's rows, and the lane quad of a key
// combines its eight accumulators by DPP exchanges that form exactly the
// reference's trees: the hadd tree ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)) for
// keys below kv_len & ~3, eng_hsum256 ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7))
// above it (fp32 addition is commutative, so every lane of the quad holds the
// same bits).  Workgroup (kv head, 64 keys); K rows staged in LDS with a row
// stride of HD + 8 words, so the quad reads of 8 consecutive keys fall on
// distinct banks.
// ---------------------------------------------------------------------------
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

template <int HD, int GM, bool ROPE>
__global__ __launch_bounds__(256) void k_attn_sc1(const float* __restrict__ q, const float* __restrict__ kc,
                                                  const int32_t* __restrict__ pos0p, int n_q, int n_kv, int max_seq,
                                                  float scale, float* __restrict__ S, ScRope ra) {
    constexpr int LD = HD + 8, E = HD / 64;
    extern __shared__ __align__(16) float sm[];
    float* ks = sm;               // [AS_KC][LD]
    float* qs = ks + AS_KC * LD;  // [GM][HD]
    const int kvh = blockIdx.x, t0 = blockIdx.y * AS_KC, tid = threadIdx.x;
    const int G = n_q / n_kv;
    const int pos = *pos0p, L = pos + 1;
    if (t0 >= L) return;  // every key of the chunk is past the row
    // ROPE units of wave tid / 64: q rows u < GM, then (if this chunk holds
    // the position) the new K row as unit GM; a wave takes u = w, w + 4, w + 8
    const int w = tid >> 6, lane = tid & 63;
    const bool has_new = ROPE && pos < t0 + AS_KC;
    const int nu = GM + (has_new ? 1 : 0);
    QkHead<HD> hu[3];
    float vv[E];
    {
        constexpr int NK = AS_KC * (HD / 4) / 256, NQ = (GM * (HD / 4) + 255) / 256;
        float4 kx[NK], qx[NQ];
#pragma unroll
        for (int k = 0; k < NK; k++) {
            const int e = tid + 256 * k, kr = e / (HD / 4), c = e % (HD / 4);
            const int t = t0 + kr < max_seq ? t0 + kr : max_seq - 1;
            kx[k] = *(const float4*)(kc + ((size_t)kvh * max_seq + t) * HD + 4 * c);
        }
        if (ROPE) {
#pragma unroll
            for (int k = 0; k < 3; k++) {
                const int u = w + 4 * k;
                if (u < GM) {
                    const int hr = u < G ? u : G - 1;  // rows past the group repeat the last head (never written)
                    qk_head_load<HD>(q + ((size_t)kvh * G + hr) * HD, ra.qn, ra.cos_tab, ra.sin_tab, pos, lane, hu[k]);
                } else if (u < nu) {
                    qk_head_load<HD>(ra.k + (size_t)kvh * HD, ra.kn, ra.cos_tab, ra.sin_tab, pos, lane, hu[k]);
#pragma unroll
                    for (int e = 0; e < E; e++) vv[e] = ra.v[(size_t)kvh * HD + lane + 64 * e];
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < NQ; k++) {
                const int e = tid + 256 * k, r = e / (HD / 4), c = e % (HD / 4);
                const int hr = r < G ? r : G - 1;  // rows past the group repeat the last head (never written)
                if (e < GM * (HD / 4)) qx[k] = *(const float4*)(q + ((size_t)kvh * G + hr) * HD + 4 * c);
            }
        }
#pragma unroll
        for (int k = 0; k < NK; k++) {
            const int e = tid + 256 * k, kr = e / (HD / 4), c = e % (HD / 4);
            *(float4*)&ks[kr * LD + 4 * c] = kx[k];
        }
        if (!ROPE) {
#pragma unroll
            for (int k = 0; k < NQ; k++) {
                const int e = tid + 256 * k;
                if (e < GM * (HD / 4)) *(float4*)&qs[4 * e] = qx[k];
            }
        }
    }
    __syncthreads();
    if (ROPE) {
        // after the barrier: the new K row replaces the chunk's (stale) copy
#pragma unroll
        for (int k = 0; k < 3; k++) {
            const int u = w + 4 * k;
            if (u >= nu) continue;  // wave-uniform
            float o[E];
            qk_head_rope<HD>(hu[k], (u < GM ? ra.qn : ra.kn) != nullptr, ra.eps, lane, o);
            if (u < GM) {
#pragma unroll
                for (int e = 0; e < E; e++) qs[u * HD + lane + 64 * e] = o[e];
            } else {
                const size_t off = ((size_t)kvh * max_seq + pos) * HD;
#pragma unroll
                for (int e = 0; e < E; e++) {
                    ks[(pos - t0) * LD + lane + 64 * e] = o[e];
                    ra.kc[off + lane + 64 * e] = o[e];
                    ra.vc[off + lane + 64 * e] = vv[e];
                }
            }
        }
        __syncthreads();
    }
    const int kq = tid >> 2, jp = tid & 3;
    float acc[GM][2];
#pragma unroll
    for (int r = 0; r < GM; r++) acc[r][0] = acc[r][1] = 0.0f;
    const float* kr = ks + kq * LD + 2 * jp;
#pragma unroll 4
    for (int i = 0; i < HD; i += 8) {
        const float2 kv = *(const float2*)(kr + i);
#pragma unroll
        for (int r = 0; r < GM; r++) {
            const float2 qv = *(const float2*)(qs + r * HD + i + 2 * jp);
            acc[r][0] = fmaf(qv.x, kv.x, acc[r][0]);
            acc[r][1] = fmaf(qv.y, kv.y, acc[r][1]);
        }
    }
    const int t = t0 + kq;
    const int n4 = L & ~3;
#pragma unroll
    for (int r = 0; r < GM; r++) {
        // hadd tree: pair sums, then (jp 0 + jp 1) and (jp 2 + jp 3), then lo + hi
        const float s = acc[r][0] + acc[r][1];
        const float u = s + fxor1(s);
        const float th = u + fxor2(u);
        // eng_hsum256: (a_j + a_{j+4}) with the quad partner two lanes away
        const float x0 = fxor2(acc[r][0]), x1 = fxor2(acc[r][1]);
        const float p = (acc[r][0] + x0) + (acc[r][1] + x1);
        const float te = p + fxor1(p);
        if (r < G && (r & 3) == jp && t < L)
            S[((size_t)kvh * G + r) * max_seq + t] = (t < n4 ? th : te) * scale;
    }
}

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
// One-token decode over long contexts: the softmax once per score row
// (k_attn_smx), then P.V spread over the chip (k_attn_pvw).
//
// k_attn_pv computes the softmax of its rows in every dim-chunk workgroup and
// runs each output's chain a = fma(p[t], v[t], a) over all keys from LDS; at
// 4096 keys its 128 workgroups spend ~39 us per layer.  Here a row's softmax
// is computed once, in the reference's order (max; exp polynomial on the
// 8-aligned keys, libm expf on the tail; eight sum lanes over t = j mod 8 and
// their eng_hsum256 tree, then the tail in order; 1 / (sum + 1e-12); p = e *
// inv, dpuf_engine.c:371-468), and written back in place.  The P.V chains,
// one per (head, dim) and in key order as before, then run on one wave per
// (kv head, DW dims): 256 workgroups at head dim 128 and DW 4, each streaming
// its 16-byte slice of every V row and its heads' probabilities through an
// LDS ring by direct-to-LDS loads several chunks ahead, so a chain step waits
// for neither memory nor another wave.
// ---------------------------------------------------------------------------

// Softmax of one score row of a one-token decode step, in place: row r =
// blockIdx.x of S (stride max_seq), length pos + 1 <= 64 SEG, SMX_NT threads.
// The row is read once, into registers: exps of the 8-aligned part go to LDS as [8][8 SEG] (lane j's
// elements t = j mod 8 in order, zero past the row: adding +0.0 leaves the
// non-negative sums exact), the tail's (< 8) to a small array.  Wave 0 runs
// the eight sum chains register-fed, chain j on lanes 8j .. 8j+7 in segments
// of SEG (as k_resnorm_prep), then the eng_hsum256 tree and the tail in
// order; the row is normalised from LDS and written once.
#define SMX_NT 1024  // threads per softmax row (SEG a multiple of 16)

template <int SEG>
__global__ __launch_bounds__(SMX_NT) void k_attn_smx(float* __restrict__ S, const int32_t* __restrict__ pos0p,
                                                  int max_seq) {
    constexpr int LDT = 8 * SEG + 4;  // row stride of the transposed copy
    __shared__ __align__(16) float tr[8][LDT];
    __shared__ float tail[8];
    __shared__ float red[SMX_NT / 64];
    __shared__ float part[8];
    float* row = S + (size_t)blockIdx.x * max_seq;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int L = *pos0p + 1, n8 = L & ~7;
    // zero the positions past the row that the chains read
    for (int i = tid; i < 8 * LDT; i += SMX_NT) (&tr[0][0])[i] = 0.0f;
    // the row in registers, all loads in flight at once (keys t = tid +
    // SMX_NT k, k < 64 SEG / SMX_NT, cover the 64 SEG keys of the largest row)
    constexpr int KR = 64 * SEG / SMX_NT;
    float xr[KR];
#pragma unroll
    for (int k = 0; k < KR; k++) xr[k] = row[min(tid + SMX_NT * k, L - 1)];
    float mx = -1e30f;
#pragma unroll
    for (int k = 0; k < KR; k++)
        if (tid + SMX_NT * k < L) mx = fmaxf(mx, xr[k]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) red[wv] = mx;
    __syncthreads();
    float M = red[0];
#pragma unroll
    for (int i = 1; i < SMX_NT / 64; i++) M = fmaxf(M, red[i]);
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int t = tid + SMX_NT * k;
        if (t < n8) tr[t & 7][t >> 3] = exp_poly(xr[k] - M);
        else if (t < L) tail[t - n8] = expf_libc(xr[k] - M);
    }
    __syncthreads();
    if (tid < 64) {
        const int j = tid >> 3, sg = tid & 7;
        float x[SEG];
#pragma unroll
        for (int i = 0; i < SEG / 4; i++) {
            const float4 e = *(const float4*)&tr[j][sg * SEG + 4 * i];
            x[4 * i] = e.x;
            x[4 * i + 1] = e.y;
            x[4 * i + 2] = e.z;
            x[4 * i + 3] = e.w;
        }
        float a = 0.0f;
#pragma unroll
        for (int ss = 0; ss < 8; ss++) {
            if (sg == ss) {
#pragma unroll
                for (int i = 0; i < SEG; i++) a = a + x[i];
            }
            const float prev = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(a), 0x111, 0xF, 0xF,
                                                                          false));
            if (sg == ss + 1) a = prev;
        }
        if (sg == 7) part[j] = a;
    }
    __syncthreads();
    if (tid == 0) {
        float sp = hsum8(part);
        for (int t = n8; t < L; t++) sp += tail[t - n8];  // the tail keys in order
        red[0] = 1.0f / (sp + 1e-12f);
    }
    __syncthreads();
    const float inv = red[0];
#pragma unroll
    for (int k = 0; k < KR; k++) {
        const int t = tid + SMX_NT * k;
        if (t < L) row[t] = (t < n8 ? tr[t & 7][t >> 3] : tail[t - n8]) * inv;
    }
}

#define PVW_CK 256  // keys per chunk

#define PVW_LD (PVW_CK + 4)  // LDS row stride of a chunk (rows on distinct banks)

// a = fma(p[t], v[t], a) over the first n keys of a chunk, in order; p and v
// are 16-byte aligned LDS rows.  A full chunk is unrolled in 8-key blocks,
// each block's four 16-byte reads issued three blocks ahead: at most 12 LDS
// reads are in flight, within what the LDS wait counter can express (15), so
// every wait is for exactly the block about to be used (with 16 in flight the
// compiler fell back to waiting for all of them).  A partial chunk takes the
// loop.
DEV float pvw_chunk(const float* p, const float* v, int n, float a) {
    if (n == PVW_CK) {
        constexpr int NB = PVW_CK / 8, AH = 3;
        float4 pb[AH + 1][2], vb[AH + 1][2];
#pragma unroll
        for (int k = 0; k < AH; k++)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                pb[k][i] = *(const float4*)(p + 8 * k + 4 * i);
                vb[k][i] = *(const float4*)(v + 8 * k + 4 * i);
            }
        // the schedule is pinned (the scheduler otherwise moved each block's
        // reads down to just before its FMAs): the prologue's reads, then per
        // block the next reads followed by its 8 FMAs
        __builtin_amdgcn_sched_group_barrier(0x100, 4 * AH, 0);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int cur = b % (AH + 1);
            if (b + AH < NB) {
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    pb[(b + AH) % (AH + 1)][i] = *(const float4*)(p + 8 * (b + AH) + 4 * i);
                    vb[(b + AH) % (AH + 1)][i] = *(const float4*)(v + 8 * (b + AH) + 4 * i);
                }
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                a = fmaf(pb[cur][i].x, vb[cur][i].x, a);
                a = fmaf(pb[cur][i].y, vb[cur][i].y, a);
                a = fmaf(pb[cur][i].z, vb[cur][i].z, a);
                a = fmaf(pb[cur][i].w, vb[cur][i].w, a);
            }
            __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
        }
        return a;
    }
    for (int t = 0; t < n; t++) a = fmaf(p[t], v[t], a);
    return a;
}

// Chunk c (clamped to the last one) of a k_attn_pvw workgroup into a
// producer lane's registers (producer lane pl of 128): V rows c0 + pl and
// c0 + 128 + pl, the key's 4 dims each (16 bytes); P 16-byte pieces 4 pl and
// 4 pl + 512 of the chunk's [GM][PVW_CK] block (heads past G read head G - 1,
// keys clamped into the row).
//
// Q8 (the int8 KV cache): V comes as 4 int8 per key (in r[i].x) and the lane
// also loads the V scales of its P pieces' 4 keys (r[2 + GM / 2]; every piece
// of a lane covers the same keys), so the store can write W = p * vs (the
// reference's p * v_scale, dpuf_engine.c:726-747) in p's place and V widened
// to floats (exact).
template <int HD, int GM, bool Q8>
DEV void pvw_load(const float* Vh, const float* Ph, const int8_t* Vq, const float* Vs, int c, int nck, int G,
                  int max_seq, int pl, gm_f4 (&r)[3 + GM / 2]) {
    const int c0 = (c < nck ? c : nck - 1) * PVW_CK;
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int key = min(c0 + 128 * i + pl, max_seq - 1);
        if (Q8) r[i][0] = __int_as_float(*(const int32_t*)(Vq + (size_t)key * HD));
        else r[i] = *(const gm_f4*)(Vh + (size_t)key * HD);
    }
#pragma unroll
    for (int i = 0; i < GM / 2; i++) {
        const int f = 512 * i + 4 * pl, hh = min(f / PVW_CK, G - 1), t = min(c0 + f % PVW_CK, max_seq - 4);
        r[2 + i] = *(const gm_f4*)(Ph + (size_t)hh * max_seq + t);
    }
    if (Q8) {
        const int t = min(c0 + (4 * pl) % PVW_CK, max_seq - 4);
#pragma unroll
        for (int k = 0; k < 4; k++) r[2 + GM / 2][k] = Vs[(size_t)(t + k) * (HD / 32)];
    }
}

// A producer lane's chunk into an LDS slot, V transposed to [dim][key].
template <int GM, bool Q8>
DEV void pvw_store(float (*Vt)[PVW_LD], float (*Pt)[PVW_LD], int pl, const gm_f4 (&r)[3 + GM / 2]) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int k = 128 * i + pl;
        if (Q8) {
            const int32_t b = __float_as_int(r[i][0]);
#pragma unroll
            for (int dd = 0; dd < 4; dd++) Vt[dd][k] = (float)(int8_t)(b >> (8 * dd));
        } else {
            Vt[0][k] = r[i][0];
            Vt[1][k] = r[i][1];
            Vt[2][k] = r[i][2];
            Vt[3][k] = r[i][3];
        }
    }
#pragma unroll
    for (int i = 0; i < GM / 2; i++) {
        const int f = 512 * i + 4 * pl;
        gm_f4 w = r[2 + i];
        if (Q8) {
#pragma unroll
            for (int k = 0; k < 4; k++) w[k] = w[k] * r[2 + GM / 2][k];
        }
        *(gm_f4*)&Pt[f / PVW_CK][f % PVW_CK] = w;
    }
}

// P.V of a one-token step over normalised probabilities P (row kvh * G + h
// of stride max_seq) for the G <= GM query heads of kv head blockIdx.x and
// dims 4 blockIdx.y .. + 3.  Wave 0 runs the chains, lane h * 4 + d, over
// LDS only; waves 1 and 2 produce: chunk c of PVW_CK keys is loaded into
// register set c % 4 four chunks ahead and written to LDS slot c % 2 one
// chunk ahead of its chains, one barrier per chunk.  The loop is unrolled by
// 4 so every register set index is static.
template <int HD, int GM, bool Q8>
__global__ __launch_bounds__(192) void k_attn_pvw(const float* __restrict__ P, const float* __restrict__ vc,
                                                  const int32_t* __restrict__ pos0p, int n_q, int n_kv,
                                                  int max_seq, float* __restrict__ out, DpufKvQ8 c8) {
    static_assert(GM >= 2 && GM * 4 <= 64 && GM % 2 == 0, "lane layout");
    __shared__ __align__(16) float Vt[2][4][PVW_LD];
    __shared__ __align__(16) float Pt[2][GM][PVW_LD];
    const int kvh = blockIdx.x, d0 = blockIdx.y * 4, tid = threadIdx.x, w = tid >> 6;
    const int G = n_q / n_kv, h = tid >> 2, d = tid & 3, pl = tid - 64;
    const int L = *pos0p + 1, nck = (L + PVW_CK - 1) / PVW_CK;
    const float* Vh = Q8 ? nullptr : vc + (size_t)kvh * max_seq * HD + d0;
    const int8_t* Vq = Q8 ? c8.vq + (size_t)kvh * max_seq * HD + d0 : nullptr;
    const float* Vs = Q8 ? c8.vs + (size_t)kvh * max_seq * (HD / 32) + d0 / 32 : nullptr;
    const float* Ph = P + (size_t)kvh * G * max_seq;
    gm_f4 r0[3 + GM / 2], r1[3 + GM / 2], r2[3 + GM / 2], r3[3 + GM / 2];  // native vectors: no struct copies
    if (w > 0) {
        pvw_load<HD, GM, Q8>(Vh, Ph, Vq, Vs, 0, nck, G, max_seq, pl, r0);
        pvw_load<HD, GM, Q8>(Vh, Ph, Vq, Vs, 1, nck, G, max_seq, pl, r1);
        pvw_load<HD, GM, Q8>(Vh, Ph, Vq, Vs, 2, nck, G, max_seq, pl, r2);
        pvw_load<HD, GM, Q8>(Vh, Ph, Vq, Vs, 3, nck, G, max_seq, pl, r3);
        pvw_store<GM, Q8>(Vt[0], Pt[0], pl, r0);
    }
    __syncthreads();
    float a = 0.0f;
    // chunk C is in LDS slot C & 1; producers load chunk C + 4 into RL (which
    // held chunk C) and write chunk C + 1 (in RN) to the other slot
#define PVW_STEP(C, RL, RN)                                                                           \
    {                                                                                                 \
        const int sl = (C) & 1;                                                                       \
        if (w == 0) {                                                                                 \
            if (h < G) a = pvw_chunk(&Pt[sl][h][0], &Vt[sl][d][0], min(PVW_CK, L - (C) * PVW_CK), a); \
        } else {                                                                                      \
            pvw_load<HD, GM, Q8>(Vh, Ph, Vq, Vs, (C) + 4, nck, G, max_seq, pl, RL);                   \
            pvw_store<GM, Q8>(Vt[sl ^ 1], Pt[sl ^ 1], pl, RN);                                        \
        }                                                                                             \
        __syncthreads();                                                                              \
    }
    for (int c = 0; c < nck; c += 4) {
        PVW_STEP(c, r0, r1)
        if (c + 1 >= nck) break;
        PVW_STEP(c + 1, r1, r2)
        if (c + 2 >= nck) break;
        PVW_STEP(c + 2, r2, r3)
        if (c + 3 >= nck) break;
        PVW_STEP(c + 3, r3, r0)
    }
#undef PVW_STEP
    if (w == 0 && h < G) out[(size_t)(kvh * G + h) * HD + d0 + d] = a;
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

// ---------------------------------------------------------------------------
// Small utility kernels
// ---------------------------------------------------------------------------
// ---------------------------------------------------------------------------
// CRC32 of tile bodies (reflected polynomial 0xEDB88320, init and final xor
// 0xFFFFFFFF: the check of reference dpuf_avx2.c:347-398), one workgroup per
// tile.  Thread i folds chunk i of the body with the byte table; chunk CRCs
// combine by linearity, crc(A || B) = crc(A) * x^(8 |B|) xor crc0(B) in
// GF(2)[x] / P (crc0: register started at 0), so each thread multiplies its
// chunk's CRC by x^(8 * bytes after the chunk) and the results are xor-ed.
// ---------------------------------------------------------------------------
#define CRC_POLY 0xEDB88320u

// a * b mod P for reflected CRC32 polynomials (bit 31 is x^0).
DEV uint32_t crc_mulmod(uint32_t a, uint32_t b) {
    uint32_t p = 0;
    for (int i = 0; i < 32; i++) {
        if (a & (0x80000000u >> i)) p ^= b;
        b = (b & 1u) ? (b >> 1) ^ CRC_POLY : b >> 1;  // b * x
    }
    return p;
}

// x^(8 n) mod P by square-and-multiply (x^0 = 0x80000000, x^8 = 0x00800000).
DEV uint32_t crc_xpow8(uint32_t n) {
    uint32_t r = 0x80000000u, sq = 0x00800000u;
    while (n) {
        if (n & 1u) r = crc_mulmod(r, sq);
        sq = crc_mulmod(sq, sq);
        n >>= 1;
    }
    return r;
}

__global__ __launch_bounds__(256) void k_crc_tiles(const uint8_t* __restrict__ base, const uint64_t* __restrict__ off,
                                                   const uint32_t* __restrict__ len, const uint32_t* __restrict__ want,
                                                   uint8_t* __restrict__ ok) {
    __shared__ uint32_t tab[256];
    __shared__ uint32_t red[4];
    const int tid = threadIdx.x, t = blockIdx.x;
    {
        uint32_t c = (uint32_t)tid;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? (CRC_POLY ^ (c >> 1)) : (c >> 1);
        tab[tid] = c;
    }
    __syncthreads();
    const uint8_t* body = base + off[t];
    const uint32_t L = len[t], S = (L + 255u) / 256u;
    const uint32_t b0 = min((uint32_t)tid * S, L), b1 = min(b0 + S, L);
    uint32_t c = tid == 0 ? 0xFFFFFFFFu : 0u;
    for (uint32_t i = b0; i < b1; i++) c = tab[(c ^ body[i]) & 0xFFu] ^ (c >> 8);
    c = crc_mulmod(c, crc_xpow8(L - b1));
    for (int o = 32; o > 0; o >>= 1) c ^= __shfl_xor(c, o, 64);
    if ((tid & 63) == 0) red[tid >> 6] = c;
    __syncthreads();
    if (tid == 0) {
        const uint32_t crc = (red[0] ^ red[1] ^ red[2] ^ red[3]) ^ 0xFFFFFFFFu;
        ok[t] = crc == want[t] ? 1u : 0u;
    }
}

__global__ void k_fill_f32(float* p, size_t n, float v) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}
__global__ void k_fill_zero_u32(uint32_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}
__global__ void k_fill_zero_u8(uint8_t* p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}
__global__ void k_zero_rows(float* out, int ld, int r0, int r1) {
    const int m = blockIdx.x;
    for (int r = r0 + threadIdx.x; r < r1; r += blockDim.x) out[(size_t)m * ld + r] = 0.0f;
}
__global__ void k_capture(int H, const float* h, const float* hn, float* cap) {
    const int m = blockIdx.x;
    for (int i = threadIdx.x; i < H; i += blockDim.x) cap[(size_t)m * H + i] = h[(size_t)m * H + i] + hn[(size_t)m * H + i];
}

// Device reductions over a logit row, in two launches: RED_NB workgroups each
// reduce a contiguous slice (float4 loads, all of a thread's loads in flight,
// wave shuffles, one LDS step) into a partial, then one wave merges the
// partials.  Scratch: RED_NB partials of 8 bytes.
#define RED_NB 64

// Top-2 with multiplicity (the reference's sequential b1/b2 scan,
// dpuf_engine.c:2101-2110, is order independent), then the early-exit
// decision b1 - b2 >= thr (thr > 0).
DEV void top2_take(float v, float& b1, float& b2) {
    if (v > b1) {
        b2 = b1;
        b1 = v;
    } else if (v > b2) {
        b2 = v;
    }
}

DEV void top2_merge(float& b1, float& b2, float c1, float c2) {
    if (b1 >= c1) {
        b2 = fmaxf(b2, c1);
    } else {
        b2 = fmaxf(c2, b1);
        b1 = c1;
    }
}

// First maximum (dpuf-cli.c:1997-2004: `if (x[i] > best)` from best = x[0]):
// the larger value, the smaller index on ties; every partial starts from
// (x[0], 0), so a NaN x[0] gives 0 as the reference does and other NaNs are
// never taken.
DEV void amax_merge(float& bv, int& bi, float v, int i) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__global__ __launch_bounds__(256) void k_red_part(const float* __restrict__ x, int n, int argmax, float2* part) {
    __shared__ float2 wp[4];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // h leading elements up to 16-byte alignment (workgroup 0), then float4
    // slices, then the tail (the last workgroup)
    const int h = min((int)((16u - ((uint32_t)(uintptr_t)x & 15u)) & 15u) >> 2, n);
    const int n4 = (n - h) >> 2, per = (n4 + RED_NB - 1) / RED_NB;
    const int c0 = blockIdx.x * per, c1 = min(c0 + per, n4);
    const float4* x4 = (const float4*)(x + h);
    float a = argmax ? x[0] : -1e30f, b = -1e30f;  // argmax: (value, index bits); top-2: (b1, b2)
    int ai = 0;
    if (blockIdx.x == 0 && tid < h) {
        if (argmax) amax_merge(a, ai, x[tid], tid);
        else top2_take(x[tid], a, b);
    }
    constexpr int U = 4;
    for (int c = c0 + tid; c < c1; c += 256 * U) {
        float4 v[U];
#pragma unroll
        for (int k = 0; k < U; k++) v[k] = c + 256 * k < c1 ? x4[c + 256 * k] : make_float4(-1e30f, -1e30f, -1e30f, -1e30f);
#pragma unroll
        for (int k = 0; k < U; k++) {
            if (c + 256 * k >= c1) continue;
            const int e = h + 4 * (c + 256 * k);
            if (argmax) {
                amax_merge(a, ai, v[k].x, e);
                amax_merge(a, ai, v[k].y, e + 1);
                amax_merge(a, ai, v[k].z, e + 2);
                amax_merge(a, ai, v[k].w, e + 3);
            } else {
                top2_take(v[k].x, a, b);
                top2_take(v[k].y, a, b);
                top2_take(v[k].z, a, b);
                top2_take(v[k].w, a, b);
            }
        }
    }
    if (blockIdx.x == RED_NB - 1)  // the n % 4 tail
        for (int e = h + 4 * n4 + tid; e < n; e += 256) {
            if (argmax) amax_merge(a, ai, x[e], e);
            else top2_take(x[e], a, b);
        }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float oa = __shfl_xor(a, o, 64);
        if (argmax) {
            const int oi = __shfl_xor(ai, o, 64);
            amax_merge(a, ai, oa, oi);
        } else {
            const float ob = __shfl_xor(b, o, 64);
            top2_merge(a, b, oa, ob);
        }
    }
    if (lane == 0) wp[w] = argmax ? make_float2(a, __int_as_float(ai)) : make_float2(a, b);
    __syncthreads();
    if (tid == 0) {
        float2 r = wp[0];
        for (int k = 1; k < 4; k++) {
            if (argmax) {
                int ri = __float_as_int(r.y);
                amax_merge(r.x, ri, wp[k].x, __float_as_int(wp[k].y));
                r.y = __int_as_float(ri);
            } else {
                top2_merge(r.x, r.y, wp[k].x, wp[k].y);
            }
        }
        part[blockIdx.x] = r;
    }
}

// One wave: merge the RED_NB partials; argmax writes the index to out[0],
// the top-2 check writes out[0] = (thr > 0 && b1 - b2 >= thr).
__global__ __launch_bounds__(64) void k_red_fin(const float2* __restrict__ part, int argmax, float thr,
                                                int32_t* out) {
    const int lane = threadIdx.x;
    // lanes past the partials hold the identity (argmax: partial 0 again)
    float2 r = lane < RED_NB ? part[lane] : (argmax ? part[0] : make_float2(-1e30f, -1e30f));
    int ri = __float_as_int(r.y);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float oa = __shfl_xor(r.x, o, 64);
        if (argmax) {
            const int oi = __shfl_xor(ri, o, 64);
            amax_merge(r.x, ri, oa, oi);
        } else {
            const float ob = __shfl_xor(r.y, o, 64);
            top2_merge(r.x, r.y, oa, ob);
        }
    }
    if (lane == 0) *out = argmax ? ri : ((thr > 0.0f && (r.x - r.y) >= thr) ? 1 : 0);
}


// ---------------------------------------------------------------------------
// Standalone-entry helpers: FWHT-only transform and slab (re)packing of the
// reference's multi-token activation layout ([n_blk][8 words][6 tokens] per
// 6-token slab, dpuf_avx2.c:2390-2447).
// ---------------------------------------------------------------------------
__global__ void k_fwht_sign(int K, const float* __restrict__ x, const uint8_t* __restrict__ sign, float* __restrict__ out) {
    const int m = blockIdx.x;
    for (int blk = threadIdx.x; blk < (K >> 6); blk += blockDim.x) {
        float v[64];
        const float* src = x + (size_t)m * K + 64 * blk;
#pragma unroll
        for (int i = 0; i < 64; i++) v[i] = src[i];
        if (sign) {
#pragma unroll
            for (int bb = 0; bb < 8; bb++) {
                const uint32_t sb = sign[8 * blk + bb];
#pragma unroll
                for (int k = 0; k < 8; k++)
                    if ((sb >> k) & 1u) v[8 * bb + k] = -v[8 * bb + k];
            }
        }
        fwht64(v);
        float* dst = out + (size_t)m * K + 64 * blk;
#pragma unroll
        for (int i = 0; i < 64; i++) dst[i] = v[i];
    }
}

// rows [mc][K] -> one slab; only token lanes j < mc are written.
__global__ void k_slab_pack(int mc, int K, DpufPrep rows, int32_t* __restrict__ sq, float* __restrict__ ss,
                            int32_t* __restrict__ sm) {
    const int nb = K >> 5;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < nb * 8 * mc; i += gridDim.x * blockDim.x) {
        const int j = i % mc, g = (i / mc) % 8, b = i / (8 * mc);
        sq[b * 48 + g * 6 + j] = *(const int32_t*)(rows.q + (size_t)j * K + b * 32 + g * 4);
        if (g == 0) {
            ss[b * 6 + j] = rows.s[(size_t)j * nb + b];
            sm[b * 6 + j] = rows.m[(size_t)j * nb + b];
        }
    }
}

// slabs of M tokens -> rows [M][K].
__global__ void k_slab_unpack(int M, int K, const int32_t* __restrict__ sq, const float* __restrict__ ss,
                              const int32_t* __restrict__ sm, DpufPrep rows) {
    const int nb = K >> 5;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < M * nb * 8; i += gridDim.x * blockDim.x) {
        const int g = i % 8, b = (i / 8) % nb, m = i / (8 * nb);
        const int slab = m / 6, j = m % 6;
        const size_t base = (size_t)slab * nb;
        const int32_t w4 = sq[(base + b) * 48 + g * 6 + j];
        *(int32_t*)(rows.q + (size_t)m * K + b * 32 + g * 4) = w4;
        if (rows.h) {
            uint32_t a, c;
            i8x4_to_h((uint32_t)w4, a, c);
            *(uint2*)(rows.h + (size_t)m * K + b * 32 + g * 4) = make_uint2(a, c);
        }
        if (g == 0) {
            rows.s[(size_t)m * nb + b] = ss[(base + b) * 6 + j];
            rows.m[(size_t)m * nb + b] = sm[(base + b) * 6 + j];
        }
    }
}

// ---------------------------------------------------------------------------
// extern "C" layer
// ---------------------------------------------------------------------------
#define ST(s) ((hipStream_t)(s))

extern "C" {

int32_t dpuf_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}
const char* dpuf_hip_error_string(void) { return g_err == hipSuccess ? "" : g_err_msg; }
int32_t dpuf_hip_ok(void) { return g_err == hipSuccess; }
void dpuf_hip_clear_error(void) { g_err = hipSuccess; g_err_msg[0] = 0; }

void* dpuf_hip_malloc(size_t bytes) {
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes ? bytes : 256);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}
void dpuf_hip_free(void* p) { if (p) CK(hipFree(p)); }
void* dpuf_hip_host_alloc(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}
void* dpuf_hip_host_alloc_io(size_t bytes) {
    void* p = nullptr;
    if (hipHostMalloc(&p, bytes ? bytes : 64, hipHostMallocCoherent) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}
void dpuf_hip_host_free(void* p) { if (p) CK(hipHostFree(p)); }
void* dpuf_hip_stream_create(void) {
    hipStream_t s = nullptr;
    CK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    return (void*)s;
}
void dpuf_hip_stream_destroy(void* s) { if (s) CK(hipStreamDestroy(ST(s))); }
int32_t dpuf_hip_sync(void* s) {
    CK(hipStreamSynchronize(ST(s)));
    return g_err == hipSuccess ? 0 : -1;
}
void dpuf_hip_h2d(void* dst, const void* src, size_t n, void* s) {
    if (n) CK(hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, ST(s)));
}
void dpuf_hip_d2h(void* dst, const void* src, size_t n, void* s) {
    if (n) CK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, ST(s)));
}
void dpuf_hip_d2d(void* dst, const void* src, size_t n, void* s) {
    if (n) CK(hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToDevice, ST(s)));
}
void dpuf_hip_fill_zero(void* dst, size_t n, void* s) {
    if (!n) return;
    if ((n & 3) == 0 && ((uintptr_t)dst & 3) == 0) {
        size_t w = n / 4;
        int blocks = (int)((w + 255) / 256 < 4096 ? (w + 255) / 256 : 4096);
        hipLaunchKernelGGL(k_fill_zero_u32, dim3(blocks), dim3(256), 0, ST(s), (uint32_t*)dst, w);
    } else {
        int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
        hipLaunchKernelGGL(k_fill_zero_u8, dim3(blocks), dim3(256), 0, ST(s), (uint8_t*)dst, n);
    }
    LAUNCHED("k_fill_zero");
}
void dpuf_hip_fill_f32(float* dst, size_t n, float v, void* s) {
    if (!n) return;
    int blocks = (int)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
    hipLaunchKernelGGL(k_fill_f32, dim3(blocks), dim3(256), 0, ST(s), dst, n, v);
    LAUNCHED("k_fill_f32");
}

void* dpuf_hip_event_create(void) {
    hipEvent_t e = nullptr;
    CK(hipEventCreate(&e));
    return (void*)e;
}
void dpuf_hip_event_destroy(void* e) { if (e) CK(hipEventDestroy((hipEvent_t)e)); }
void dpuf_hip_event_record(void* e, void* s) { CK(hipEventRecord((hipEvent_t)e, ST(s))); }
void dpuf_hip_event_sync(void* e) { CK(hipEventSynchronize((hipEvent_t)e)); }
float dpuf_hip_event_elapsed_ms(void* a, void* b) {
    float ms = 0.0f;
    CK(hipEventSynchronize((hipEvent_t)b));
    CK(hipEventElapsedTime(&ms, (hipEvent_t)a, (hipEvent_t)b));
    return ms;
}

int32_t dpuf_hip_capture_begin(void* s) {
    hipError_t e = hipStreamBeginCapture(ST(s), hipStreamCaptureModeThreadLocal);
    note(e, "hipStreamBeginCapture");
    return e == hipSuccess ? 0 : -1;
}
void* dpuf_hip_capture_end(void* s) {
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipStreamEndCapture(ST(s), &g);
    note(e, "hipStreamEndCapture");
    if (e != hipSuccess || !g) return nullptr;
    e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    note(e, "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    return e == hipSuccess ? (void*)ge : nullptr;
}
int32_t dpuf_hip_graph_launch(void* g, void* s) {
    hipError_t e = hipGraphLaunch((hipGraphExec_t)g, ST(s));
    note(e, "hipGraphLaunch");
    return e == hipSuccess ? 0 : -1;
}
void dpuf_hip_graph_destroy(void* g) { if (g) (void)hipGraphExecDestroy((hipGraphExec_t)g); }

void dpuf_hip_embed(void* s, DpufDevW w, const int32_t* ids, int32_t M, const float* embeds, float* out,
                    const int32_t* pos_src, int32_t* pos_dst, int32_t* serial_dst) {
    int threads = (w.cols >> 6) < 256 ? (w.cols >> 6) : 256;
    threads = (threads + 63) & ~63;
    hipLaunchKernelGGL(k_embed, dim3(M), dim3(threads), 0, ST(s), w, ids, embeds, out, pos_src, pos_dst,
                       serial_dst);
    LAUNCHED("k_embed");
}

// Copies a step's result words (early-exit flag, argmax token, error word)
// to host memory with vector stores, so the host reads them after the
// stream drains without a copy; the flag is 0 when no top-2 check ran.
__global__ void k_publish(const int32_t* __restrict__ words, int flag_valid, int32_t* host) {
    if (threadIdx.x == 0) {
        host[0] = flag_valid ? words[0] : 0;
        host[1] = words[1];
        host[2] = words[2];
    }
}

void dpuf_hip_publish(void* s, const int32_t* words, int32_t flag_valid, int32_t* host) {
    hipLaunchKernelGGL(k_publish, dim3(1), dim3(64), 0, ST(s), words, flag_valid, host);
    LAUNCHED("k_publish");
}

void dpuf_hip_resnorm_prep(void* s, int32_t M, int32_t H, const float* h, const float* res, float* h_out,
                           const float* w, float eps, int32_t n_prep, const uint8_t* const* signs,
                           const DpufPrep* preps, float* xn_out) {
    if (res && !h_out) {
        note(hipErrorInvalidValue, "dpuf_hip_resnorm_prep: a residual add needs h_out");
        return;
    }
    PrepSet ps;
    memset(&ps, 0, sizeof ps);
    ps.n = n_prep;
    for (int i = 0; i < n_prep; i++) {
        ps.sign[i] = signs[i];
        ps.p[i] = preps[i];
        if (M == 1) ps.p[i].h = NULL;  // the one-row GEMV reads q only
    }
    const int threads = H / 16;  // H is a multiple of 1024 or 64 * 16 * k; checked at engine create
    const size_t lds = (size_t)8 * ((H >> 3) + 4) * sizeof(float);
    // register-fed chains for the widths with a 16-byte-aligned segment
    // (8 * (H / 8 + 4) floats per row keeps segments of 16, 32, 64 aligned)
    // four workgroups per row when the row splits into quarters of whole
    // 16-lane rows of blocks (and no normalised copy is asked for)
    const bool split = M <= 16 && H % 256 == 0 && !xn_out && !(res && h_out == h);
    auto k = split ? (H == 4096   ? k_resnorm_prep<64, 4>
                      : H == 2048 ? k_resnorm_prep<32, 4>
                      : H == 1024 ? k_resnorm_prep<16, 4>
                                  : k_resnorm_prep<0, 4>)
                   : (H == 4096   ? k_resnorm_prep<64, 1>
                      : H == 2048 ? k_resnorm_prep<32, 1>
                      : H == 1024 ? k_resnorm_prep<16, 1>
                                  : k_resnorm_prep<0, 1>);
    hipLaunchKernelGGL(k, dim3(M, split ? 4 : 1), dim3(threads), lds, ST(s), H, h, res, h_out, w, eps, ps, xn_out);
    LAUNCHED("k_resnorm_prep");
}

void dpuf_hip_prep(void* s, int32_t M, int32_t K, const float* x, const uint8_t* sign, DpufPrep p) {
    const int quads = K / 16;
    if (M == 1) p.h = NULL;
    // one wave per workgroup: the rows' loads spread over many CUs
    hipLaunchKernelGGL(k_prep, dim3((quads + 63) / 64, M), dim3(64), 0, ST(s), K, x, sign, p);
    LAUNCHED("k_prep");
}

void dpuf_hip_swiglu_prep(void* s, int32_t M, int32_t I, const float* gate, const float* up, float dz,
                          const uint8_t* sign, DpufPrep p) {
    if (M == 1) p.h = NULL;
    hipLaunchKernelGGL(k_swiglu_prep, dim3((I + 255) / 256, M), dim3(64), 0, ST(s), I, gate, up, dz, sign, p);
    LAUNCHED("k_swiglu_prep");
}

void dpuf_hip_relayout(void* s, const uint8_t* src, const uint64_t* offs, int32_t n_groups, int32_t n_blk,
                       int32_t mode, uint8_t* dst) {
    const size_t total = (size_t)n_groups * n_blk * 8;
    const int blocks = (int)((total + 255) / 256 < 65536 ? (total + 255) / 256 : 65536);
    hipLaunchKernelGGL(k_relayout, dim3(blocks), dim3(256), 0, ST(s), src, offs, n_groups, n_blk, (int)(mode == 14),
                       dst);
    LAUNCHED("k_relayout");
}

typedef void (*MvKernel)(MvArgs);

static int g_mv_max_wg = 0;  // test/tuning cap on GEMV / K-split GEMM workgroups

// Compute units of the current device (cached; 1 when the query fails).
static int dpuf_hip_cu_count() {
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 1;
    }
    return n_cu;
}

void dpuf_hip_set_gemv_max_wg(int32_t n) { g_mv_max_wg = n > 0 ? n : 0; }

// Device error word of the current API call on this thread (see MvArgs::err).
static thread_local int32_t* g_err_word = NULL;

void dpuf_hip_bind_error_word(int32_t* d_word) { g_err_word = d_word; }

// Workgroups of one k_mv instance the device holds at once (occupancy x CUs),
// cached per (instance, block size, LDS size).
static int mv_capacity(MvKernel k, int threads, size_t lds) {
    static int n_cu = 0;
    static MvKernel c_k[64];
    static int c_t[64], c_cap[64], c_n = 0;
    static size_t c_lds[64];
    for (int i = 0; i < c_n; i++)
        if (c_k[i] == k && c_t[i] == threads && c_lds[i] == lds) return c_cap[i];
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 1;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int cap = per_cu * n_cu;
    if (c_n < 64) {
        c_k[c_n] = k;
        c_t[c_n] = threads;
        c_lds[c_n] = lds;
        c_cap[c_n++] = cap;
    }
    return cap;
}

// Picks the instance for S steps per group: one round per group with
// NL = 1..4 steps per loader wave and at most 15 loader waves (S <= 60),
// otherwise 8 loader waves x 2 steps per round with the activations loaded
// per round.  The block has one more wave, the chain wave.
extern "C++" {
template <int MODE>
static void mv_pick(int S, MvKernel& k, MvKernel& k1, int& nl, int& nw) {
    if (S <= 16 - MV_NC) {
        nl = 1;
        k = k_mv<1, true, false, MODE>;
        k1 = k_mv<1, true, true, MODE>;
    } else if (S <= 2 * (16 - MV_NC)) {
        nl = 2;
        k = k_mv<2, true, false, MODE>;
        k1 = k_mv<2, true, true, MODE>;
    } else if (S <= 3 * (16 - MV_NC)) {
        nl = 3;
        k = k_mv<3, true, false, MODE>;
        k1 = k_mv<3, true, true, MODE>;
    } else if (S <= 4 * (16 - MV_NC) && MV_HOIST48) {
        nl = 4;
        k = k_mv<4, true, false, MODE>;
        k1 = k_mv<4, true, true, MODE>;
    } else {
        nl = 2;
        k = k_mv<2, false, false, MODE>;
        k1 = k_mv<2, false, true, MODE>;
    }
    nw = k == k_mv<2, false, false, MODE> ? 8 : (S + nl - 1) / nl;
}
}

// The launch plan of a one-row GEMV over n_jobs jobs of one mode: the
// instances (persistent, one group per workgroup), loader waves nw, the
// workgroup prefix sums wb[0..n_jobs] and the most groups of one workgroup.
// Returns the total group count (0: nothing to launch).
static int mv_plan(int n_jobs, const int* n_groups, int K, int mode, MvKernel& k, MvKernel& k1, int& nw, int* wb,
                   int& most) {
    const int n_blk = K >> 5, S = (n_blk + 7) >> 3;
    int nl;
    if (mode == 13) mv_pick<13>(S, k, k1, nl, nw);
    else if (mode == 14) mv_pick<14>(S, k, k1, nl, nw);
    else mv_pick<12>(S, k, k1, nl, nw);
    (void)nl;
    const int threads_p = (nw + MV_NC) * 64;  // + the chain waves
    const size_t buf = (size_t)8 * (n_blk + 2) * 8;
    int total = 0;
    for (int i = 0; i < n_jobs; i++) total += n_groups[i];
    if (total <= 0) return 0;
    // one group per workgroup when the chip holds all of them at once,
    // otherwise persistent workgroups with chain waves
    int cap1 = mv_capacity(k1, nw * 64, buf);
    if (g_mv_max_wg > 0 && cap1 > g_mv_max_wg) cap1 = g_mv_max_wg;
    int cap = total <= cap1 ? total : mv_capacity(k, threads_p, MV_NBUF * buf);
    if (g_mv_max_wg > 0 && cap > g_mv_max_wg) cap = g_mv_max_wg;
    int grid = 0;
    most = 1;
    wb[0] = 0;
    for (int i = 0; i < n_jobs; i++) {
        int nwg = n_groups[i];
        if (total > cap && nwg > 0) {
            nwg = (int)((long long)cap * n_groups[i] / total);
            if (nwg < 1) nwg = 1;
        }
        if (nwg > 0 && (n_groups[i] + nwg - 1) / nwg > most) most = (n_groups[i] + nwg - 1) / nwg;
        grid += nwg;
        wb[i + 1] = grid;
    }
    return total;
}

// One launch over jobs of one mode.
static void mv_launch(void* s, MvArgs& A, const int* n_groups, int mode) {
    const int n_blk = A.K >> 5;
    MvKernel k, k1;
    int nw, most;
    if (mv_plan(A.n_jobs, n_groups, A.K, mode, k, k1, nw, A.wb, most) == 0) return;
    const int grid = A.wb[A.n_jobs];
    const size_t buf = (size_t)8 * (n_blk + 2) * 8;
    if (!g_err_word) {
        note(hipErrorInvalidValue, "dpuf_hip_gemv: no device error word bound");
        return;
    }
    A.err = g_err_word;
    A.nbuf = most < MV_NBUF ? most : MV_NBUF;
    A.nc = most > 1 ? MV_NC : 0;
    const int threads = (nw + A.nc) * 64;
    const size_t lds = (size_t)A.nbuf * buf;
    hipLaunchKernelGGL(A.nc ? k : k1, dim3(grid), dim3(threads), lds, ST(s), A);
    LAUNCHED("k_mv");
}

// The producer-fed instance with nl steps per loader wave.
extern "C++" {
template <int MODE>
static MvKernel mv_fed_of(int nl) {
    return nl == 1 ? k_mv<1, true, true, MODE, true>
         : nl == 2 ? k_mv<2, true, true, MODE, true>
         : nl == 3 ? k_mv<3, true, true, MODE, true>
                   : k_mv<4, true, true, MODE, true>;
}
}
static MvKernel mv_fed_kernel(int mode, int nl) {
    return mode == 13 ? mv_fed_of<13>(nl) : mode == 14 ? mv_fed_of<14>(nl) : mv_fed_of<12>(nl);
}

// SwiGLU + dead zone + prep of gate / up [I] (up NULL: the plain prep of
// gate) and the one-row GEMV of job over them in one launch: producer
// workgroups first (k_mv's producer-fed mode),
// the MV_FLAG_COPIES copies flags[64 c + p] of producer p set to the step serial *serial when its share is out.
// Only for a plan of one group per workgroup with the activations held
// (every workgroup resident at once, weights issued before the wait);
// returns -1 without launching otherwise.
int32_t dpuf_hip_swiglu_gemv(void* s, int32_t I, const float* gate, const float* up, float dz, const uint8_t* sign,
                             const DpufGemvJob* job, int32_t* flags, const int32_t* serial) {
    const int mode = job->w.mode;
    if ((mode != 12 && mode != 13 && mode != 14) || job->w.cols != I || I <= 0 || I % 64 || !flags || !serial)
        return -1;
    const int n_blk = I >> 5, S = (n_blk + 7) >> 3;
    if (S > (MV_HOIST48 ? 4 : 3) * (16 - MV_NC)) return -1;  // activations loaded per round: no such mode
    const int ng = job->g1 - job->g0 > 0 ? job->g1 - job->g0 : 0;
    MvKernel k, k1;
    int nw, most, wb[4] = {0, 0, 0, 0};
    if (mv_plan(1, &ng, I, mode, k, k1, nw, wb, most) == 0 || most != 1) return -1;
    const int threads = nw * 64, np = (I / 4 + threads - 1) / threads;
    if (np > 64) return -1;
    const int nl = S <= 16 - MV_NC ? 1 : S <= 2 * (16 - MV_NC) ? 2 : S <= 3 * (16 - MV_NC) ? 3 : 4;
    MvKernel kf = mv_fed_kernel(mode, nl);
    const size_t lds = (size_t)8 * (n_blk + 2) * 8;
    if (ng > mv_capacity(kf, threads, lds)) return -1;  // every GEMV workgroup resident at once
    if (!g_err_word) {
        note(hipErrorInvalidValue, "dpuf_hip_swiglu_gemv: no device error word bound");
        return -1;
    }
    MvArgs A;
    memset(&A, 0, sizeof A);
    A.n_jobs = 1;
    A.K = I;
    A.j[0].g = job->w.g;
    A.j[0].out = job->out;
    A.j[0].g0 = job->g0;
    A.j[0].g1 = job->g1;
    A.j[0].rows = job->w.rows;
    A.j[0].x = job->p;
    A.j[0].x.h = NULL;
    A.wb[0] = wb[0];
    A.wb[1] = wb[1];
    A.err = g_err_word;
    A.nbuf = 1;
    A.nc = 0;
    A.np = np;
    A.pI = I;
    A.pg = gate;
    A.pu = up;
    A.pdz = dz;
    A.psign = sign;
    A.pflag = flags;
    A.pep = serial;
    hipLaunchKernelGGL(kf, dim3(np + wb[1]), dim3(threads), lds, ST(s), A);
    LAUNCHED("k_mv");
    return 0;
}

static void gm_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs, float* zo, int32_t zld, int32_t z0,
                      int32_t z1);

typedef void (*GmKernel)(GmArgs);

// Workgroups of a K-split GEMM instance the device holds at once.
static int gm_capacity(GmKernel k, int threads) {
    static int n_cu = 0;
    static GmKernel c_k[4];
    static int c_cap[4], c_n = 0;
    for (int i = 0; i < c_n; i++)
        if (c_k[i] == k) return c_cap[i];
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 1;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, threads, 0) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int cap = per_cu * n_cu;
    if (c_n < 4) {
        c_k[c_n] = k;
        c_cap[c_n++] = cap;
    }
    return cap;
}

void dpuf_hip_gemv_zero(void* s, int32_t M, const DpufGemvJob* job, int32_t r0, int32_t r1) {
    if (M == 1) {
        dpuf_hip_gemv(s, 1, 1, job, NULL, 0.0f);
        if (r1 > r0) dpuf_hip_zero_rows(s, 1, job->out, job->ldo, r0, r1);
        return;
    }
    gm_launch(s, M, 1, job, job->out, job->ldo, r0, r1);
}

int32_t dpuf_hip_warm_add(DpufWarm* wm, int32_t n_jobs, const DpufGemvJob* jobs, int32_t r0, int32_t nr) {
    if (!wm || n_jobs < 1 || n_jobs > 3 || nr < 1 || r0 < 0 || wm->n_jobs + n_jobs > DPUF_WARM_JOBS) return 0;
    const int mode = jobs[0].w.mode;
    int ng[3] = {0, 0, 0};
    for (int j = 0; j < n_jobs; j++) {
        if (jobs[j].w.mode != mode || jobs[j].w.cols != jobs[0].w.cols) return 0;
        ng[j] = jobs[j].g1 - jobs[j].g0 > 0 ? jobs[j].g1 - jobs[j].g0 : 0;
    }
    MvKernel k, k1;
    int nw, most, wb[4];
    if (mv_plan(n_jobs, ng, jobs[0].w.cols, mode, k, k1, nw, wb, most) == 0 || r0 >= most) return 0;
    if (nr > most - r0) nr = most - r0;
    const int gb = (jobs[0].w.cols >> 5) * dpuf_grp_unit(mode);
    for (int j = 0; j < n_jobs; j++) {
        DpufWarmJob& J = wm->j[wm->n_jobs + j];
        J.p = jobs[j].w.g + (size_t)jobs[j].g0 * gb;
        J.n_groups = ng[j];
        J.group_bytes = gb;
        J.wb = wb[j];
        J.nwg = wb[j + 1] - wb[j];
        J.r0 = r0;
        J.nr = nr;
    }
    wm->n_jobs += n_jobs;
    return 1;
}

void dpuf_hip_gemv(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs, const int32_t* skip_flag,
                   float fill) {
    // jobs of different modes go to one launch per mode, in order of first use
    for (int i = 0; i < n_jobs; i++) {
        const int mode = jobs[i].w.mode;
        if (mode != 12 && mode != 13 && mode != 14) {
            note(hipErrorInvalidValue, "dpuf_hip_gemv: matrix mode other than 12, 13, 14");
            return;
        }
        bool seen = false;
        for (int j = 0; j < i; j++) seen = seen || jobs[j].w.mode == mode;
        if (seen) continue;
        DpufGemvJob sub[3];
        int n = 0;
        for (int j = i; j < n_jobs; j++)
            if (jobs[j].w.mode == mode) sub[n++] = jobs[j];
        if (M > 1) {
            gm_launch(s, M, n, sub, NULL, 0, 0, 0);
            continue;
        }
        MvArgs A;
        memset(&A, 0, sizeof A);
        int ng[3] = {0, 0, 0};
        A.n_jobs = n;
        A.K = sub[0].w.cols;
        for (int j = 0; j < n; j++) {
            A.j[j].g = sub[j].w.g;
            A.j[j].out = sub[j].out;
            A.j[j].g0 = sub[j].g0;
            A.j[j].g1 = sub[j].g1;
            A.j[j].rows = sub[j].w.rows;
            A.j[j].x = sub[j].p;
            ng[j] = sub[j].g1 - sub[j].g0 > 0 ? sub[j].g1 - sub[j].g0 : 0;
        }
        A.skip_flag = skip_flag;
        A.fill = fill;
        mv_launch(s, A, ng, mode);
    }
}

// The M > 1 GEMM; rows [z0, z1) of zo are zeroed by the same launch.
static void gm_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs, float* zo, int32_t zld, int32_t z0,
                      int32_t z1) {
    {
        GmArgs G;
        memset(&G, 0, sizeof G);
        int t = 0;
        G.n_jobs = n_jobs;
        G.K = jobs[0].w.cols;
        G.M = M;
        for (int i = 0; i < n_jobs; i++) {
            G.j[i].g = jobs[i].w.g;
            G.j[i].g0 = jobs[i].g0;
            G.j[i].g1 = jobs[i].g1;
            G.j[i].rows = jobs[i].w.rows;
            G.j[i].h = jobs[i].p.h;
            if ((long long)M * G.K >= (1ll << 30)) {
                note(hipErrorInvalidValue, "dpuf_hip_gemv: M * K must stay below 2^30");
                return;
            }
            if (!jobs[i].p.h) {
                note(hipErrorInvalidValue, "dpuf_hip_gemv: M > 1 needs the fp16 activations (DpufPrep.h)");
                return;
            }
            G.j[i].s = jobs[i].p.s;
            G.j[i].m = jobs[i].p.m;
            G.j[i].out = jobs[i].out;
            G.j[i].ldo = jobs[i].ldo;
            G.tb[i] = t;
            const int ng = jobs[i].g1 - jobs[i].g0;
            t += ng > 0 ? (ng + 8 * GM_RF - 1) / (8 * GM_RF) : 0;
        }
        G.tb[n_jobs] = t;
        if (zo && z1 > z0) {
            G.zo = zo;
            G.zld = zld;
            G.z0 = z0;
            G.z1 = z1;
            G.zt = (z1 - z0 + 63) / 64;
        }
        if (t + G.zt <= 0) return;
        const int n_blk = G.K >> 5;
        const int mode = jobs[0].w.mode;  // one mode per launch (dpuf_hip_gemv groups them)
        long long gmax = 0;
        for (int i = 0; i < n_jobs; i++) gmax = gmax > jobs[i].g1 ? gmax : jobs[i].g1;
        if (mode == 12 && M <= 16 && n_blk <= 128 && gmax * n_blk * 144 < 0xFFFFFFFFll) {
            // one 16-token tile, K <= 4096: persistent K-split workgroups,
            // each job's share of the chip in proportion to its fragments
            const int NR = n_blk <= 32 ? 1 : n_blk <= 64 ? 2 : 4;
            GmKernel k = NR == 1 ? k_gemm_skp<1> : NR == 2 ? k_gemm_skp<2> : k_gemm_skp<4>;
            int cap = gm_capacity(k, 64 * (SK_NP + SK_NC));
            if (g_mv_max_wg > 0 && cap > g_mv_max_wg) cap = g_mv_max_wg;
            int nfr[3], ftot = 0;
            for (int i = 0; i < n_jobs; i++) {
                const int ng = jobs[i].g1 - jobs[i].g0;
                nfr[i] = ng > 0 ? (ng + 1) / 2 : 0;
                ftot += nfr[i];
            }
            int wgs = 0;
            for (int i = 0; i < n_jobs; i++) {
                G.tb[i] = wgs;
                int nw = ftot > 0 ? (int)(((long long)cap * nfr[i] + ftot - 1) / ftot) : 0;
                nw = nw < 1 ? 1 : nw;
                wgs += nfr[i] > 0 ? (nw < nfr[i] ? nw : nfr[i]) : 0;
            }
            G.tb[n_jobs] = wgs;
            hipLaunchKernelGGL(k, dim3(wgs + G.zt), dim3(64 * (SK_NP + SK_NC)), 0, ST(s), G);
            LAUNCHED("k_gemm_skp");
            return;
        }
        if (mode == 12 && M <= 16) {
            // one 16-token tile: the K-split kernel, one workgroup per 16 rows
            int f = 0;
            for (int i = 0; i < n_jobs; i++) {
                G.tb[i] = f;
                const int ng = jobs[i].g1 - jobs[i].g0;
                f += ng > 0 ? (ng + 1) / 2 : 0;
            }
            G.tb[n_jobs] = f;
            hipLaunchKernelGGL(k_gemm_sk, dim3(f + G.zt), dim3(64 * (SK_NP + SK_NC)), 0, ST(s), G);
            LAUNCHED("k_gemm_sk");
            return;
        }
        // a multiple of 8 row tiles keeps a row tile's token tiles on one XCD
        const int gx = (t + G.zt + 7) & ~7;
        G.gy = (M + 16 * GM_TT - 1) / (16 * GM_TT);
        const dim3 grid = GM_XCD ? dim3(gx * G.gy) : dim3(gx, G.gy);
        // modes 13 / 14 take this kernel at every M (the K-split kernels
        // are mode 12 only)
        if (mode == 13)
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 13>), grid, dim3(256), 0, ST(s), G);
        else if (mode == 14)
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 14>), grid, dim3(256), 0, ST(s), G);
        else
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 12>), grid, dim3(256), 0, ST(s), G);
        LAUNCHED("k_gemm_mfma");
    }
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
// not apply.
static int32_t attn_split(void* s, int32_t M, int32_t lmax, const float* q, const float* kc, const float* vc,
                          float* out, float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd,
                          int32_t max_seq, float scale, const uint8_t* o_sign, DpufPrep op, int32_t* prepped,
                          const ScRope* rope) {
    if (prepped) *prepped = 0;
    if (rope && M != 1) return -1;
    if (n_kv <= 0 || n_q % n_kv || n_q / n_kv > 32 || (hd != 64 && hd != 128 && hd != 256)) return -1;
    if (lmax > max_seq) lmax = max_seq;
    const int G = n_q / n_kv;
    // scores: up to 32 q rows (queries x group heads) per workgroup
    const int qt1 = 32 / G < M ? 32 / G : M;
    const dim3 g1(n_kv, (M + qt1 - 1) / qt1, (lmax + AS_KC - 1) / AS_KC);
    const size_t lds1 = (size_t)(AS_KC + 32) * (hd + 4) * 4;
    // softmax + P.V: R = qt2 * G rows of lcap probabilities in LDS; about 8
    // rows per workgroup keeps >= 32 dims per P.V chain group, so the
    // softmax each dim chunk repeats stays small next to P.V
    const int lcap = (lmax + 7) & ~7;
    const size_t budget = 112 * 1024;
    int qt2 = 8 / G > 1 ? 8 / G : 1;
    if (qt2 > M) qt2 = M;
    while (qt2 > 1 && (size_t)qt2 * G * lcap * 4 > budget) qt2--;
    if ((size_t)qt2 * G * lcap * 4 > budget) return -1;
    const int R = qt2 * G;
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
            return 0;
        }
    }
    // one-token decode with an even group: softmax once per row, then the
    // wide P.V (one wave per kv head and 4 dims)
    {
        // chain segments of the softmax: 8 SEG positions per sum lane cover
        // keys up to 64 SEG
        const int segs[7] = {16, 32, 48, 64, 80, 96, 128};
        int seg = 0;
        for (int i = 0; i < 7 && !seg; i++)
            if (64 * segs[i] >= lmax) seg = segs[i];
        if (M == 1 && (G & 1) == 0 && G <= 8 && seg) {
            const int gm = G <= 2 ? 2 : G <= 4 ? 4 : 8;
            const dim3 gp(n_kv, hd / 4);
#define SMX_LAUNCH(SG)                                                                                            \
    if (seg == SG) hipLaunchKernelGGL(k_attn_smx<SG>, dim3(n_q), dim3(SMX_NT), 0, ST(s), scores, pos0p, max_seq);
#define SC1_LAUNCH(HDV, GMV)                                                                                      \
    {                                                                                                             \
        const dim3 g1s(n_kv, (lmax + AS_KC - 1) / AS_KC);                                                         \
        const size_t l1s = (size_t)(AS_KC * (HDV + 8) + GMV * HDV) * 4;                                           \
        if (rope)                                                                                                 \
            hipLaunchKernelGGL((k_attn_sc1<HDV, GMV, true>), g1s, dim3(256), l1s, ST(s), q, kc, pos0p, n_q, n_kv, \
                               max_seq, scale, scores, *rope);                                                    \
        else                                                                                                      \
            hipLaunchKernelGGL((k_attn_sc1<HDV, GMV, false>), g1s, dim3(256), l1s, ST(s), q, kc, pos0p, n_q,      \
                               n_kv, max_seq, scale, scores, ScRope{});                                           \
    }
#define PVW_LAUNCH(HDV)                                                                                           \
    if (gm == 2) SC1_LAUNCH(HDV, 2) else if (gm == 4) SC1_LAUNCH(HDV, 4) else SC1_LAUNCH(HDV, 8)                  \
    SMX_LAUNCH(16) SMX_LAUNCH(32) SMX_LAUNCH(48) SMX_LAUNCH(64) SMX_LAUNCH(80) SMX_LAUNCH(96) SMX_LAUNCH(128)  \
    if (gm == 2)                                                                                                  \
        hipLaunchKernelGGL((k_attn_pvw<HDV, 2, false>), gp, dim3(192), 0, ST(s), scores, vc, pos0p, n_q, n_kv,  \
                           max_seq, out, DpufKvQ8{});                                                                                  \
    else if (gm == 4)                                                                                             \
        hipLaunchKernelGGL((k_attn_pvw<HDV, 4, false>), gp, dim3(192), 0, ST(s), scores, vc, pos0p, n_q, n_kv,  \
                           max_seq, out, DpufKvQ8{});                                                                                  \
    else                                                                                                          \
        hipLaunchKernelGGL((k_attn_pvw<HDV, 8, false>), gp, dim3(192), 0, ST(s), scores, vc, pos0p, n_q, n_kv,  \
                           max_seq, out, DpufKvQ8{});
            if (hd == 64) {
                PVW_LAUNCH(64)
            } else if (hd == 128) {
                PVW_LAUNCH(128)
            } else {
                PVW_LAUNCH(256)
            }
#undef PVW_LAUNCH
#undef SC1_LAUNCH
#undef SMX_LAUNCH
            LAUNCHED("k_attn_split_wide");
            return 0;
        }
    }
    if (rope) return -1;
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
    return 0;
}

int32_t dpuf_hip_attn_split(void* s, int32_t M, int32_t lmax, const float* q, const float* kc, const float* vc,
                            float* out, float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd,
                            int32_t max_seq, float scale, const uint8_t* o_sign, DpufPrep op, int32_t* prepped) {
    return attn_split(s, M, lmax, q, kc, vc, out, scores, pos0p, n_q, n_kv, hd, max_seq, scale, o_sign, op, prepped,
                      NULL);
}

int32_t dpuf_hip_attn_decode_rope(void* s, int32_t lmax, float* q, const float* k, const float* v, const float* qn,
                                  const float* kn, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                                  float* vc, float* out, float* scores, const int32_t* pos0p, int32_t n_q,
                                  int32_t n_kv, int32_t hd, int32_t max_seq, float scale) {
    const ScRope r = {k, v, qn, kn, eps, cos_tab, sin_tab, kc, vc};
    DpufPrep none;
    memset(&none, 0, sizeof none);
    return attn_split(s, 1, lmax, q, kc, vc, out, scores, pos0p, n_q, n_kv, hd, max_seq, scale, NULL, none, NULL, &r);
}

void dpuf_hip_attn(void* s, int32_t M, const float* q, const float* kc, const float* vc, float* out, float* scores,
                   const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq, float scale) {
    const int groups = n_q / n_kv;
    hipLaunchKernelGGL(k_attn, dim3(M, n_kv, (groups + 1) / 2), dim3(256), (size_t)2 * hd * sizeof(float), ST(s), q,
                       kc, vc, out, scores, pos0, n_q, n_kv, hd, max_seq, scale);
    LAUNCHED("k_attn");
}

void dpuf_hip_attn_q8(void* s, int32_t M, int32_t lmax, const float* q, DpufKvQ8 c8, float* out, float* scores,
                      const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq, float scale) {
    const int G = n_q / n_kv;
    if (lmax > max_seq) lmax = max_seq;
    const size_t lds1 = (size_t)G * hd * 4 + (size_t)Q8_SCK * hd + (size_t)Q8_SCK * (hd / 32) * 4;
    hipLaunchKernelGGL(k_attn_q8_sc, dim3(n_kv, (lmax + Q8_SCK - 1) / Q8_SCK, M), dim3(256), lds1, ST(s), q, c8,
                       scores, pos0, n_q, n_kv, hd, max_seq, scale);
    // one token, groups of 2, 4 or 8: the softmax once per row and P.V on one
    // chain wave per (kv head, 4 dims), as for the fp32 cache, with W = p *
    // v_scale and V widened in the producers
    if (M == 1 && (G & 1) == 0 && G <= 8) {
        const int segs[7] = {16, 32, 48, 64, 80, 96, 128};
        int seg = 0;
        for (int i = 0; i < 7 && !seg; i++)
            if (64 * segs[i] >= lmax) seg = segs[i];
        if (seg) {
            const int gm = G <= 2 ? 2 : G <= 4 ? 4 : 8;
            const dim3 gp(n_kv, hd / 4);
#define SMXQ(SG) \
    if (seg == SG) hipLaunchKernelGGL(k_attn_smx<SG>, dim3(n_q), dim3(SMX_NT), 0, ST(s), scores, pos0, max_seq);
            SMXQ(16) SMXQ(32) SMXQ(48) SMXQ(64) SMXQ(80) SMXQ(96) SMXQ(128)
#undef SMXQ
#define PVWQ(HDV)                                                                                                  \
    do {                                                                                                           \
        if (gm == 2)                                                                                               \
            hipLaunchKernelGGL((k_attn_pvw<HDV, 2, true>), gp, dim3(192), 0, ST(s), scores, nullptr, pos0, n_q, n_kv, \
                               max_seq, out, c8);                                                                  \
        else if (gm == 4)                                                                                          \
            hipLaunchKernelGGL((k_attn_pvw<HDV, 4, true>), gp, dim3(192), 0, ST(s), scores, nullptr, pos0, n_q, n_kv, \
                               max_seq, out, c8);                                                                  \
        else                                                                                                       \
            hipLaunchKernelGGL((k_attn_pvw<HDV, 8, true>), gp, dim3(192), 0, ST(s), scores, nullptr, pos0, n_q, n_kv, \
                               max_seq, out, c8);                                                                  \
    } while (0)
            if (hd == 64) PVWQ(64);
            else if (hd == 128) PVWQ(128);
            else PVWQ(256);
#undef PVWQ
            LAUNCHED("k_attn_q8_sc/k_attn_smx/k_attn_pvw<q8>");
            return;
        }
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
            return;
        }
#undef PVQ
    }
    // rows too long for LDS: softmax in memory, P.V per (token, kv head, pair)
    const size_t lds2 = 2 * 32768 + (size_t)2 * 2 * (hd / 32) * (32768 / hd) * 4;
    hipLaunchKernelGGL(k_attn_q8, dim3(M, n_kv, (G + 1) / 2), dim3(256), lds2, ST(s), c8, out, scores, pos0,
                       n_q, n_kv, hd, max_seq);
    LAUNCHED("k_attn_q8_sc/k_attn_q8");
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
    return 0;
}

void dpuf_hip_crc_tiles(void* s, const uint8_t* base, const uint64_t* off, const uint32_t* len,
                        const uint32_t* want, uint8_t* ok, int32_t n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_crc_tiles, dim3(n), dim3(256), 0, ST(s), base, off, len, want, ok);
    LAUNCHED("k_crc_tiles");
}

void dpuf_hip_zero_rows(void* s, int32_t M, float* out, int32_t ld, int32_t r0, int32_t r1) {
    if (r1 <= r0) return;
    hipLaunchKernelGGL(k_zero_rows, dim3(M), dim3(256), 0, ST(s), out, ld, r0, r1);
    LAUNCHED("k_zero_rows");
}

void dpuf_hip_capture(void* s, int32_t M, int32_t H, const float* h, const float* hn, float* cap) {
    hipLaunchKernelGGL(k_capture, dim3(M), dim3(256), 0, ST(s), H, h, hn, cap);
    LAUNCHED("k_capture");
}

void dpuf_hip_topcheck(void* s, const float* logits, int32_t n, float thr, int32_t* flag, void* scratch) {
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), logits, n, 0, (float2*)scratch);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)scratch, 0, thr, flag);
    LAUNCHED("k_red_part/k_red_fin (top-2 check)");
}

void dpuf_hip_argmax(void* s, const float* logits, int32_t V, int32_t* out, void* scratch) {
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), logits, V, 1, (float2*)scratch);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)scratch, 1, 0.0f, out);
    LAUNCHED("k_red_part/k_red_fin (argmax)");
}

// The allocation-free reduction entry's partials: one file-scope array per
// device, RED_NB float2 (512 bytes), held until the process ends.  Host code
// never passes the array's name to a kernel (in host code it is a stand-in,
// not a device address): each device's address comes from
// hipGetSymbolAddress, taken once per device with that device current.
static __device__ __align__(256) float2 scratch[RED_NB];
#define RED_MAX_DEVICES 64
static void* g_scratch_ptr[RED_MAX_DEVICES];
static std::mutex g_scratch_mu;

static float2* scratch_on_current_device(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= RED_MAX_DEVICES) {
        note(hipErrorInvalidDevice, "dpuf_hip_reduce_noalloc: no usable current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            note(e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return (float2*)g_scratch_ptr[dev];
}

int32_t dpuf_hip_reduce_noalloc(const float* x, int32_t n, int32_t mode, float thr, int32_t* out, void* s) {
    float2* part = scratch_on_current_device();
    if (!part) return -6;
    // every partial slot is written by its workgroup before k_red_fin reads
    // it, so nothing from an earlier call needs clearing
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), x, n, mode, part);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)part, mode, mode ? 0.0f : thr, out);
    LAUNCHED("k_red_part/k_red_fin (allocation-free)");
    return g_err == hipSuccess ? 0 : -6;
}

void dpuf_hip_fwht_sign(void* s, int32_t M, int32_t K, const float* x, const uint8_t* sign, float* out) {
    int threads = (K >> 6) < 256 ? (K >> 6) : 256;
    threads = (threads + 63) & ~63;
    hipLaunchKernelGGL(k_fwht_sign, dim3(M), dim3(threads), 0, ST(s), K, x, sign, out);
    LAUNCHED("k_fwht_sign");
}

void dpuf_hip_slab_pack(void* s, int32_t mc, int32_t K, DpufPrep rows, int32_t* sq, float* ss, int32_t* sm) {
    hipLaunchKernelGGL(k_slab_pack, dim3(64), dim3(256), 0, ST(s), mc, K, rows, sq, ss, sm);
    LAUNCHED("k_slab_pack");
}

void dpuf_hip_slab_unpack(void* s, int32_t M, int32_t K, const int32_t* sq, const float* ss, const int32_t* sm,
                          DpufPrep rows) {
    hipLaunchKernelGGL(k_slab_unpack, dim3(256), dim3(256), 0, ST(s), M, K, sq, ss, sm, rows);
    LAUNCHED("k_slab_unpack");
}

}  // extern "C"
