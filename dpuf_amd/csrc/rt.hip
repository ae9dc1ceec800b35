// rt.hip -- gfx950 runtime layer of the DPUF engine: error state, memory,
// streams, events and graphs, and the small kernels of the token loop
// (embedding, residual RMSNorm + prep, prep, SwiGLU + prep, weight relayout,
// CRC of tiles, fills, logit reductions, FWHT / slab helpers).
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

#include <mutex>

// ---------------------------------------------------------------------------
// Error bookkeeping
// ---------------------------------------------------------------------------
// First HIP error of the current API call on this thread: every entry point
// of the library clears it on entry (dpuf_hip_clear_error) and reports it on
// exit, so one failed call does not fail the next one or another thread's.
static thread_local hipError_t g_err = hipSuccess;
static thread_local char g_err_msg[256];

void dpuf_note(hipError_t e, const char* what) {
    if (e != hipSuccess && g_err == hipSuccess) {
        g_err = e;
        snprintf(g_err_msg, sizeof g_err_msg, "%s: %s", what, hipGetErrorString(e));
    }
}

// ---------------------------------------------------------------------------
// Embedding (reference dpuf_embed_qr_hadamard4_packed_f32, dpuf_avx2.c:2738-2783,
// and embed_qr_had_asym_impl, dpuf_avx2.c:3154-3207, for modes 13 / 14)
// grid: M rows; thread per 64-column block.
// ---------------------------------------------------------------------------
// ids (and pos_src) may sit in fine-grained host memory that the host wrote
// just before the launch: system-scope loads read them past every cache.
// Workgroup 0 copies the step's start position to pos_dst in device memory,
// where the kernels after it read it, and the step serial the host put next
// to it (pos_src[1]) to serial_dst.  Rows with a negative id copy their
// hidden state from embeds: device memory (plain float4 loads), or, with
// emb_host set, fine-grained host memory the host filled just before the
// launch (system-scope 8-byte loads, like the ids).
__global__ void k_embed(DpufDevW w, const int32_t* __restrict__ ids, const float* __restrict__ embeds,
                        int emb_host, float* __restrict__ out, const int32_t* pos_src, int32_t* pos_dst,
                        int32_t* serial_dst) {
    const int m = blockIdx.x;
    const int H = w.cols, n_blk = H >> 5;
    float* dst = out + (size_t)m * H;
    if (pos_dst && m == 0 && threadIdx.x == 0)
        *pos_dst = __hip_atomic_load(pos_src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (serial_dst && m == 0 && threadIdx.x == 0)
        *serial_dst = __hip_atomic_load(pos_src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int id = ids ? __hip_atomic_load(ids + m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : -1;
    if (embeds && id < 0 && emb_host) {
        // H is a multiple of 64: H / 2 words, all in flight at once with
        // blockDim.x = 256 and H <= 4096 (the loop covers any H)
        const uint64_t* src = (const uint64_t*)(embeds + (size_t)m * H);
        uint64_t* dst8 = (uint64_t*)dst;
        const int n8 = H >> 1, T = blockDim.x;
        for (int i0 = threadIdx.x; i0 < n8; i0 += 8 * T) {
            uint64_t v[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                v[k] = i0 + k * T < n8 ? __hip_atomic_load(src + i0 + k * T, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_SYSTEM)
                                       : 0ull;
#pragma unroll
            for (int k = 0; k < 8; k++)
                if (i0 + k * T < n8) dst8[i0 + k * T] = v[k];
        }
        return;
    }
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

// Row blockIdx.y of rows ldx apart (one row: gridDim.y = 1), its partials at
// part + RED_NB blockIdx.y.
__global__ __launch_bounds__(256) void k_red_part(const float* __restrict__ x, int n, int argmax, float2* part,
                                                  int ldx) {
    x += (size_t)blockIdx.y * ldx;
    part += (size_t)blockIdx.y * RED_NB;
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
// Row blockIdx.x's partials (part + RED_NB blockIdx.x) to out[blockIdx.x]; with
// host set, argmax also stores the index to host[blockIdx.x] (fine-grained
// host memory the caller reads after the stream drains).
__global__ __launch_bounds__(64) void k_red_fin(const float2* __restrict__ part, int argmax, float thr,
                                                int32_t* out, int32_t* host) {
    part += (size_t)blockIdx.x * RED_NB;
    out += blockIdx.x;
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
    if (lane == 0) {
        *out = argmax ? ri : ((thr > 0.0f && (r.x - r.y) >= thr) ? 1 : 0);
        if (host && argmax) host[blockIdx.x] = ri;
    }
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

void dpuf_hip_embed(void* s, DpufDevW w, const int32_t* ids, int32_t M, const float* embeds, int32_t emb_host,
                    float* out, const int32_t* pos_src, int32_t* pos_dst, int32_t* serial_dst) {
    int threads = (w.cols >> 6) < 256 ? (w.cols >> 6) : 256;
    threads = (threads + 63) & ~63;
    // host-memory rows: 256 threads put every 8-byte load of a row in flight at once
    if (embeds && emb_host) threads = 256;
    hipLaunchKernelGGL(k_embed, dim3(M), dim3(threads), 0, ST(s), w, ids, embeds, (int)(emb_host != 0), out,
                       pos_src, pos_dst, serial_dst);
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

// The LM-head reductions finished by one workgroup from the partials the
// GEMV's chains wrote (dpuf_hip_gemv_red), merged in any order.
DEV lm4 lm_block_merge(const lm4* __restrict__ part, int n) {  // 256 threads; the result in thread 0
    __shared__ lm4 sh[4];
    lm4 p = lm_part_init();
    for (int i = threadIdx.x; i < n; i += 256) p = lm_part_merge(p, part[i]);
    p = lm_part_wave(p);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = p;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int k = 1; k < 4; k++) p = lm_part_merge(p, sh[k]);
    return p;
}

// Zone-A check over the zone rows' partials: *flag = (thr > 0 && top-1 -
// top-2 >= thr) (dpuf_engine.c:2091-2136), *zone = the merged partial.
__global__ __launch_bounds__(256) void k_lm_zone(const lm4* __restrict__ part, int n, float thr, int32_t* flag,
                                                 lm4* zone) {
    const lm4 p = lm_block_merge(part, n);
    if (threadIdx.x == 0) {
        *flag = (thr > 0.0f && (p[0] - p[1]) >= thr) ? 1 : 0;
        *zone = p;
    }
}

// The row's first maximum (dpuf-cli.c:1997-2004), then the step's result
// words to host as k_publish does.  Without zone: over the n partials.  With
// zone (an early-exit step, the flag in words[0]): the zone's merged
// partial and, when the flag is set, the filled rows (fill from fill_row on;
// fill_row < 0: none) in place of the n partials of the other rows.  A NaN
// logit 0 gives 0 (the reference's scan starts from x[0]).  words = {flag,
// token, error word}; the token goes to words[1].
__global__ __launch_bounds__(256) void k_lm_argmax_publish(const lm4* __restrict__ part, int n,
                                                           const lm4* __restrict__ zone, float fill, int fill_row,
                                                           const float* __restrict__ x0, int32_t* words,
                                                           int flag_valid, int32_t* host) {
    const int32_t flag = zone ? words[0] : 0;  // uniform
    lm4 p = flag ? lm_part_init() : lm_block_merge(part, n);
    if (threadIdx.x == 0) {
        if (zone) p = lm_part_merge(p, *zone);
        if (flag && fill_row >= 0) p = lm_part_take(p, fill, fill_row);
        const float v0 = *x0;
        const int32_t tok = v0 != v0 ? 0 : __float_as_int(p[3]);
        words[1] = tok;
        host[0] = flag_valid ? flag : 0;
        host[1] = tok;
        host[2] = words[2];
    }
}

void dpuf_hip_lm_zone(void* s, const void* part, int32_t n, float thr, int32_t* flag, void* zone) {
    hipLaunchKernelGGL(k_lm_zone, dim3(1), dim3(256), 0, ST(s), (const lm4*)part, n, thr, flag, (lm4*)zone);
    LAUNCHED("k_lm_zone");
}

void dpuf_hip_lm_argmax_publish(void* s, const void* part, int32_t n, const void* zone, float fill, int32_t fill_row,
                                const float* x0, int32_t* words, int32_t flag_valid, int32_t* host) {
    hipLaunchKernelGGL(k_lm_argmax_publish, dim3(1), dim3(256), 0, ST(s), (const lm4*)part, n, (const lm4*)zone,
                       fill, fill_row, x0, words, flag_valid, host);
    LAUNCHED("k_lm_argmax_publish");
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


// Compute units of the current device (cached; 1 when the query fails).
int dpuf_hip_cu_count(void) {
    static int n_cu = 0;
    if (n_cu == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 1;
    }
    return n_cu;
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
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), logits, n, 0, (float2*)scratch, 0);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)scratch, 0, thr, flag, nullptr);
    LAUNCHED("k_red_part/k_red_fin (top-2 check)");
}

void dpuf_hip_argmax(void* s, const float* logits, int32_t V, int32_t* out, void* scratch) {
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), logits, V, 1, (float2*)scratch, 0);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)scratch, 1, 0.0f, out, nullptr);
    LAUNCHED("k_red_part/k_red_fin (argmax)");
}

void dpuf_hip_argmax_rows(void* s, const float* logits, int32_t V, int32_t n, int32_t* out, int32_t* host,
                          void* scratch) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB, n), dim3(256), 0, ST(s), logits, V, 1, (float2*)scratch, V);
    hipLaunchKernelGGL(k_red_fin, dim3(n), dim3(64), 0, ST(s), (const float2*)scratch, 1, 0.0f, out, host);
    LAUNCHED("k_red_part/k_red_fin (argmax of rows)");
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
    hipLaunchKernelGGL(k_red_part, dim3(RED_NB), dim3(256), 0, ST(s), x, n, mode, part, 0);
    hipLaunchKernelGGL(k_red_fin, dim3(1), dim3(64), 0, ST(s), (const float2*)part, mode, mode ? 0.0f : thr, out,
                       nullptr);
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
