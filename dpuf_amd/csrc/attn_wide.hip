// attn_wide.hip -- one-token decode over long contexts: the scores kernel
// with every thread working (k_attn_sc1, optionally with the QK-norm, RoPE
// and KV store of the token), the softmax once per score row (k_attn_smx)
// and the P.V chains spread over the chip (k_attn_pvw), for the fp32 and
// int8 caches.
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

// V rows that the workgroups after the n_rows softmax rows of a launch read
// into the L2 of their XCD for the P.V launch after it: with n_kv a multiple
// of 8, every chain workgroup of kv head k runs on XCD k % 8 (workgroup b of
// a launch runs on XCD b % 8, and k_attn_pvd's linear id is y n_kv + k), so
// the warm-up workgroups on XCD x read rows [0, L) of kv heads x, x + 8, ...
// (rb bytes per row, base: the V cache of kv head 0).  base NULL: no warm-up.
struct SmxWarm {
    const uint8_t* base;
    int rb, n_kv, n_rows;
};

DEV void smx_warm(const SmxWarm& W, int L, int max_seq) {
    const int id = blockIdx.x, xc = id & 7;
    const int first = W.n_rows + ((xc - W.n_rows) & 7);  // the first warm-up workgroup on XCD xc
    const int r = (id - first) >> 3, nx = ((int)gridDim.x - first + 7) >> 3;
    const size_t per = (size_t)L * W.rb;  // bytes of one kv head's rows [0, L), a multiple of 16
    const size_t lo = (per * r / nx) & ~(size_t)15, hi = r + 1 == nx ? per : (per * (r + 1) / nx) & ~(size_t)15;
    uint32_t acc = 0;
    for (int k = xc; k < W.n_kv; k += 8) {
        const uint8_t* p0 = W.base + (size_t)k * max_seq * W.rb;
        for (size_t o = lo + 16 * (size_t)threadIdx.x; o < hi; o += 16 * 8 * (size_t)blockDim.x) {
            uint4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const size_t oo = o + (size_t)i * 16 * blockDim.x;
                v[i] = oo + 16 <= hi ? *(const uint4*)(p0 + oo) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 8; i++) acc ^= v[i].x ^ v[i].w;
        }
    }
    asm volatile("" ::"v"(acc));  // the loaded values count as used: the reads stay
}

template <int SEG>
__global__ __launch_bounds__(SMX_NT) void k_attn_smx(float* __restrict__ S, const int32_t* __restrict__ pos0p,
                                                  int max_seq, SmxWarm W) {
    constexpr int LDT = 8 * SEG + 4;  // row stride of the transposed copy
    __shared__ __align__(16) float tr[8][LDT];
    __shared__ float tail[8];
    __shared__ float red[SMX_NT / 64];
    __shared__ float part[8];
    const int L = *pos0p + 1, n8 = L & ~7;
    if ((int)blockIdx.x >= W.n_rows) {
        smx_warm(W, L, max_seq);
        return;
    }
    float* row = S + (size_t)blockIdx.x * max_seq;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
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
// each block's four 16-byte reads issued three blocks ahead; scheduling
// regions of one block each keep the reads there (a pinned group schedule
// of the whole chunk ran as fast but took the compiler half a minute per
// instance).  A partial chunk takes the loop.
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
        // one scheduling region per block (the scheduler otherwise moved each
        // block's reads down to just before its FMAs): the prologue's reads,
        // then per block the next reads followed by its 8 FMAs
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int cur = b % (AH + 1);
            if (b + AH < NB) {
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    pb[(b + AH) % (AH + 1)][i] = *(const float4*)(p + 8 * (b + AH) + 4 * i);
                    vb[(b + AH) % (AH + 1)][i] = *(const float4*)(v + 8 * (b + AH) + 4 * i);
                }
            }
#pragma unroll
            for (int i = 0; i < 2; i++) {
                a = fmaf(pb[cur][i].x, vb[cur][i].x, a);
                a = fmaf(pb[cur][i].y, vb[cur][i].y, a);
                a = fmaf(pb[cur][i].z, vb[cur][i].z, a);
                a = fmaf(pb[cur][i].w, vb[cur][i].w, a);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return a;
    }
    for (int t = 0; t < n; t++) a = fmaf(p[t], v[t], a);
    return a;
}

// Keys t .. t + 3 of a probability row of max_seq entries (t a multiple of
// 4): one 16-byte load, or at the row's end element by element with keys past
// it clamped to its last one (their values are never used; the keys before
// them keep their own values whatever max_seq % 4 is).
DEV gm_f4 pv_piece(const float* row, int t, int max_seq) {
    if (t + 4 <= max_seq) return *(const gm_f4*)(row + t);
    gm_f4 r;
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = row[min(t + k, max_seq - 1)];
    return r;
}

// The int8 cache's V scales of keys t .. t + 3 (one per 32 dims, HD / 32 per
// key), clamped as pv_piece.
template <int HD>
DEV gm_f4 pv_scales(const float* Vs, int t, int max_seq) {
    gm_f4 r;
#pragma unroll
    for (int k = 0; k < 4; k++) r[k] = Vs[(size_t)min(t + k, max_seq - 1) * (HD / 32)];
    return r;
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
        const int f = 512 * i + 4 * pl, hh = min(f / PVW_CK, G - 1);
        r[2 + i] = pv_piece(Ph + (size_t)hh * max_seq, c0 + f % PVW_CK, max_seq);
    }
    if (Q8) r[2 + GM / 2] = pv_scales<HD>(Vs, c0 + (4 * pl) % PVW_CK, max_seq);
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
// k_attn_pvd: P.V of a one-token step for groups of G = 2 or 4 query heads,
// the same chains as k_attn_pvw (a = fma(p[t], v[t], a) over the keys in
// order, one per (head, dim)) with a quarter of its LDS reads per key.
//
// The chain wave's lane (h, j) = (lane / DW, lane % DW), DW = 64 / G, runs
// the chain of head h and dim d0 + j, so every 16-lane row belongs to one
// head.  Per 16 keys a lane reads its dim's transposed V row (four 16-byte
// LDS reads) and ONE probability, p[h][t + lane % 16]; key t + i takes p from
// lane i of the row through the DPP row_newbcast source of v_fmac_f32 (data
// movement only: one instruction and one rounding per key, as fmaf).  The
// chain is bound by instruction issue (a dependent v_fmac 4.6 cycles, a
// 64-lane ds_read_b128 ~11), so five reads per 16 keys instead of eight.
//
// Two producer waves stream chunks of PVD_CK keys into a 3-slot LDS ring two
// chunks ahead of the chain (register sets loaded five chunks ahead); the
// chain's reads run on into the next chunk, which is complete since the
// barrier before, so no pipeline restart per chunk.  Q8: V arrives as int8
// (widened, exact) and the producers store W = p * vs (the reference's
// p * v_scale, dpuf_engine.c:726-747) in p's place, vs the V scale of the
// WG's 32-dim block.
// ---------------------------------------------------------------------------
#define PVD_CK 256  // keys per chunk
#define PVD_AH 3    // 16-key groups read ahead by the chain
#define PVD_LD (PVD_CK + 4)  // LDS row stride (rows on distinct banks)
#ifndef PVD_SMX_WARM
#define PVD_SMX_WARM 1  // V warmed by the softmax launch (n_kv a multiple of 8)
#endif

template <int G, bool Q8>
struct PvdShape {
    static constexpr int DW = 64 / G;            // dims per workgroup
    static constexpr int LPK = DW / 4;           // producer lanes per key (4 dims each)
    static constexpr int KPI = 128 / LPK;        // keys per producer load instruction
    static constexpr int NV = PVD_CK / KPI;      // V loads per producer lane per chunk
    static constexpr int NP = G * PVD_CK / 512;  // P pieces (4 keys) per producer lane per chunk
    static constexpr int NR = NV + NP + (Q8 ? NP : 0);
};

template <int HD, int G, bool Q8>
DEV void pvd_load(const float* Vh, const int8_t* Vq, const float* Vs, const float* Ph, int c, int nck, int max_seq,
                  int pl, gm_f4 (&r)[PvdShape<G, Q8>::NR]) {
    using S = PvdShape<G, Q8>;
    const int c0 = (c < nck ? c : nck - 1) * PVD_CK;
#pragma unroll
    for (int i = 0; i < S::NV; i++) {
        const size_t key = (size_t)min(c0 + S::KPI * i + pl / S::LPK, max_seq - 1);
        const int dd = 4 * (pl % S::LPK);
        if (Q8) r[i][0] = __int_as_float(*(const int32_t*)(Vq + key * HD + dd));
        else r[i] = *(const gm_f4*)(Vh + key * HD + dd);
    }
#pragma unroll
    for (int i = 0; i < S::NP; i++) {
        const int f = 512 * i + 4 * pl, t = c0 + f % PVD_CK;
        r[S::NV + i] = pv_piece(Ph + (size_t)(f / PVD_CK) * max_seq, t, max_seq);
        if (Q8) r[S::NV + S::NP + i] = pv_scales<HD>(Vs, t, max_seq);
    }
}

template <int G, bool Q8>
DEV void pvd_store(float (*Vt)[PVD_LD], float (*Pt)[PVD_LD], int pl,
                   const gm_f4 (&r)[PvdShape<G, Q8>::NR]) {
    using S = PvdShape<G, Q8>;
#pragma unroll
    for (int i = 0; i < S::NV; i++) {
        const int key = S::KPI * i + pl / S::LPK, dd = 4 * (pl % S::LPK);
        if (Q8) {
            const int32_t b = __float_as_int(r[i][0]);
#pragma unroll
            for (int k = 0; k < 4; k++) Vt[dd + k][key] = (float)(int8_t)(b >> (8 * k));
        } else {
#pragma unroll
            for (int k = 0; k < 4; k++) Vt[dd + k][key] = r[i][k];
        }
    }
#pragma unroll
    for (int i = 0; i < S::NP; i++) {
        const int f = 512 * i + 4 * pl;
        gm_f4 w = r[S::NV + i];
        if (Q8) {
#pragma unroll
            for (int k = 0; k < 4; k++) w[k] = w[k] * r[S::NV + S::NP + i][k];
        }
        *(gm_f4*)&Pt[f / PVD_CK][f % PVD_CK] = w;
    }
}

// 16 keys of a chain: a = fma(p[t + i], v[t + i], a), i ascending, p[t + i]
// from lane i of the lane's 16-lane row.  One asm block: the DPP source pr
// comes from an LDS read, never from a VALU write inside the block, so no
// wait states are needed between the instructions.
DEV float pvd_16(float pr, const float4 (&v)[4], float a) {
    asm("v_fmac_f32_dpp %0, %1, %2 row_newbcast:0 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %3 row_newbcast:1 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %4 row_newbcast:2 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %5 row_newbcast:3 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %6 row_newbcast:4 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %7 row_newbcast:5 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %8 row_newbcast:6 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %9 row_newbcast:7 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %10 row_newbcast:8 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %11 row_newbcast:9 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %12 row_newbcast:10 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %13 row_newbcast:11 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %14 row_newbcast:12 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %15 row_newbcast:13 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %16 row_newbcast:14 row_mask:0xf bank_mask:0xf\n"
        "v_fmac_f32_dpp %0, %1, %17 row_newbcast:15 row_mask:0xf bank_mask:0xf\n"
        : "+v"(a)
        : "v"(pr), "v"(v[0].x), "v"(v[0].y), "v"(v[0].z), "v"(v[0].w), "v"(v[1].x), "v"(v[1].y), "v"(v[1].z),
          "v"(v[1].w), "v"(v[2].x), "v"(v[2].y), "v"(v[2].z), "v"(v[2].w), "v"(v[3].x), "v"(v[3].y), "v"(v[3].z),
          "v"(v[3].w));
    return a;
}

// The chain over one full chunk in slot SL; the reads of the last PVD_AH
// groups' successors go to slot SN (the next chunk).  One scheduling region
// per group keeps each group's reads ahead of its FMAs.
template <int G, bool Q8, int SL, int SN>
DEV float pvd_chunk(float (*Vt)[64 / G][PVD_LD], float (*Pt)[G][PVD_LD], int h, int j,
                    int n, float a, float (&pr)[PVD_AH + 1], float4 (&vb)[PVD_AH + 1][4]) {
    constexpr int NG = PVD_CK / 16;
    static_assert(NG % (PVD_AH + 1) == 0, "the read-ahead ring index is static across chunks");
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const int cur = g % (PVD_AH + 1), ng = g + PVD_AH;
        const int ns = ng < NG ? SL : SN, no = (ng < NG ? ng : ng - NG) * 16;
        pr[ng % (PVD_AH + 1)] = Pt[ns][h][no + n];
#pragma unroll
        for (int i = 0; i < 4; i++) vb[ng % (PVD_AH + 1)][i] = *(const float4*)(&Vt[ns][j][no + 4 * i]);
        a = pvd_16(pr[cur], vb[cur], a);
        __builtin_amdgcn_sched_barrier(0);
    }
    return a;
}

// Waits until at most N vector-memory operations of this wave are in flight.
#define PVD_VMCNT(N) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory")

template <int HD, int G, bool Q8>
__global__ __launch_bounds__(192) void k_attn_pvd(const float* __restrict__ P, const float* __restrict__ vc,
                                                  const int32_t* __restrict__ pos0p, int n_kv, int max_seq,
                                                  float* __restrict__ out, DpufKvQ8 c8, DpufWarm warm) {
    using S = PvdShape<G, Q8>;
    constexpr int DW = S::DW;
    static_assert(G == 2 || G == 4, "every 16-lane row of the chain wave holds one head");
    __shared__ __align__(16) float Vt[3][DW][PVD_LD];
    __shared__ __align__(16) float Pt[3][G][PVD_LD];
    const int L = *pos0p + 1, nck = (L + PVD_CK - 1) / PVD_CK, nfull = L / PVD_CK;
    if ((int)blockIdx.y >= HD / DW) {
        // warm-up workgroups (after the chain workgroups in dispatch order)
        const int wi = ((int)blockIdx.y - HD / DW) * n_kv + (int)blockIdx.x;
        if (warm.n_wg > 0) {
            // the weight groups of the GEMVs after this launch
            warm_read(warm, wi, (int)(blockIdx.y * gridDim.x + blockIdx.x), threadIdx.x, blockDim.x);
            return;
        }
        // else the V rows past the chunks the producers load at their start
        // go into the Infinity Cache, so the producers' later loads hit there
        // instead of each of the few chain CUs pulling its slice from HBM
        const int nw = ((int)gridDim.y - HD / DW) * n_kv;
        constexpr int RB = Q8 ? HD : HD * 4;  // bytes per V row
        const uint8_t* base = Q8 ? (const uint8_t*)c8.vq : (const uint8_t*)vc;
        const int k0 = 5 * PVD_CK;
        if (L <= k0) return;
        const int kvw = wi % n_kv, part = wi / n_kv, parts = nw / n_kv;
        const size_t seg = (size_t)(L - k0) * RB, lo = seg * part / parts, hi = seg * (part + 1) / parts;
        const uint8_t* p0 = base + ((size_t)kvw * max_seq + k0) * RB;
        uint32_t acc = 0;
        for (size_t o = lo + 16 * (size_t)threadIdx.x; o < hi; o += 16 * 8 * (size_t)blockDim.x) {
            uint4 v[8];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const size_t oo = o + (size_t)k * 16 * blockDim.x;
                v[k] = oo + 16 <= hi ? *(const uint4*)(p0 + oo) : make_uint4(0, 0, 0, 0);
            }
#pragma unroll
            for (int k = 0; k < 8; k++) acc ^= v[k].x ^ v[k].w;
        }
        asm volatile("" ::"v"(acc));  // the loaded values count as used: the reads stay
        return;
    }
    const int kvh = blockIdx.x, d0 = blockIdx.y * DW, tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
    const int h = lane / DW, j = lane % DW, n = lane & 15, pl = tid - 64;
    const float* Vh = Q8 ? nullptr : vc + (size_t)kvh * max_seq * HD + d0;
    const int8_t* Vq = Q8 ? c8.vq + (size_t)kvh * max_seq * HD + d0 : nullptr;
    const float* Vs = Q8 ? c8.vs + (size_t)kvh * max_seq * (HD / 32) + d0 / 32 : nullptr;
    const float* Ph = P + (size_t)kvh * G * max_seq;
    gm_f4 r0[S::NR], r1[S::NR], r2[S::NR];  // chunks c % 3
    float pr[PVD_AH + 1];
    float4 vb[PVD_AH + 1][4];
    if (w > 0) {
        pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, 0, nck, max_seq, pl, r0);
        pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, 1, nck, max_seq, pl, r1);
        pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, 2, nck, max_seq, pl, r2);
        PVD_VMCNT(2 * S::NR);
        pvd_store<G, Q8>(Vt[0], Pt[0], pl, r0);
        pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, 3, nck, max_seq, pl, r0);
        PVD_VMCNT(2 * S::NR);
        pvd_store<G, Q8>(Vt[1], Pt[1], pl, r1);
        pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, 4, nck, max_seq, pl, r1);
    }
    __syncthreads();
    float a = 0.0f;
    if (w == 0) {
#pragma unroll
        for (int k = 0; k < PVD_AH; k++) {
            pr[k] = Pt[0][h][16 * k + n];
#pragma unroll
            for (int i = 0; i < 4; i++) vb[k][i] = *(const float4*)(&Vt[0][j][16 * k + 4 * i]);
        }
    }
    // Step C: the chain consumes chunk C (slot C % 3; its reads run on into
    // slot (C + 1) % 3, written before the previous barrier); the producers
    // store chunk C + 2 (register set (C + 2) % 3, loaded three steps ago)
    // into slot (C + 2) % 3, whose chunk C - 1 the chain finished before that
    // barrier, and load chunk C + 5 into the set.  The chain wave passes the
    // barrier without waiting for its reads in flight (they target slots
    // nobody writes in this step); the producers wait for their LDS stores.
#define PVD_STEP(C, SL, SN, RS)                                                                        \
    {                                                                                                  \
        if (w == 0) {                                                                                  \
            if ((C) < nfull) {                                                                         \
                a = pvd_chunk<G, Q8, SL, SN>(Vt, Pt, h, j, n, a, pr, vb);                              \
            } else if ((C) == nfull) {                                                                 \
                const int nn = L - (C) * PVD_CK;                                                       \
                for (int t = 0; t < nn; t++) a = fmaf(Pt[SL][h][t], Vt[SL][j][t], a);                 \
            }                                                                                          \
            __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                   \
            __builtin_amdgcn_s_barrier();                                                              \
            __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                   \
        } else {                                                                                       \
            PVD_VMCNT(S::NR);                                                                          \
            pvd_store<G, Q8>(Vt[((SL) + 2) % 3], Pt[((SL) + 2) % 3], pl, RS);                          \
            pvd_load<HD, G, Q8>(Vh, Vq, Vs, Ph, (C) + 5, nck, max_seq, pl, RS);                        \
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");                                         \
            __builtin_amdgcn_s_barrier();                                                              \
            __atomic_signal_fence(__ATOMIC_SEQ_CST);                                                   \
        }                                                                                              \
    }
    for (int c = 0; c < nck; c += 3) {
        PVD_STEP(c, 0, 1, r2)
        if (c + 1 >= nck) break;
        PVD_STEP(c + 1, 1, 2, r0)
        if (c + 2 >= nck) break;
        PVD_STEP(c + 2, 2, 0, r1)
    }
#undef PVD_STEP
    if (w == 0) out[(size_t)(kvh * G + h) * HD + d0 + j] = a;
}

// The softmax launch of a one-token step over n_q score rows; before a
// k_attn_pvd launch (groups of 2 and 4) with n_kv a multiple of 8, one
// workgroup per remaining CU (a multiple of 8) warms the V rows (base, rb
// bytes per row) into the L2 that reads them.
static void smx_launch(void* s, int seg, float* scores, const int32_t* pos0p, int max_seq, int n_q, int n_kv, int G,
                       const void* vbase, int rb) {
    SmxWarm W{nullptr, rb, n_kv, n_q};
    int nwarm = 0;
    if (PVD_SMX_WARM && (G == 2 || G == 4) && n_kv % 8 == 0 && vbase) {
        nwarm = (dpuf_hip_cu_count() - n_q) & ~7;
        if (nwarm > 0) W.base = (const uint8_t*)vbase;
        else nwarm = 0;
    }
    const dim3 g(n_q + nwarm);
#define SMX_CASE(SG) \
    if (seg == SG) hipLaunchKernelGGL(k_attn_smx<SG>, g, dim3(SMX_NT), 0, ST(s), scores, pos0p, max_seq, W);
    SMX_CASE(16) SMX_CASE(32) SMX_CASE(48) SMX_CASE(64) SMX_CASE(80) SMX_CASE(96) SMX_CASE(128)
#undef SMX_CASE
}

// The one-token P.V launch: k_attn_pvd for groups of 2 and 4, else k_attn_pvw
// (gm: its group instance, 2, 4 or 8).
template <int HD, bool Q8>
static void pv_wide_launch(void* s, int G, int gm, const float* scores, const float* vc, const int32_t* pos0p, int n_q,
                           int n_kv, int max_seq, float* out, DpufKvQ8 c8, const DpufWarm* wm) {
    // k_attn_pvd: HD / DW chain workgroups per kv head, then warm-up
    // workgroups up to about one per CU: of the GEMV weights in wm, or (when
    // the softmax launch did not warm V into the L2s) of V
    if (G == 4 || G == 2) {
        const int ns = HD / (64 / G), n_cu = dpuf_hip_cu_count();
        DpufWarm warm;
        memset(&warm, 0, sizeof warm);
        int rows = 0;
        if (wm && wm->sink && wm->n_jobs > 0 && n_cu > n_kv * ns + 8) {
            warm = *wm;
            warm.n_wg = (n_cu - n_kv * ns) & ~7;
            rows = (warm.n_wg + n_kv - 1) / n_kv;
        } else if (!(PVD_SMX_WARM && n_kv % 8 == 0 && n_cu - n_q >= 8)) {
            rows = (n_cu / n_kv > ns ? n_cu / n_kv : ns) - ns;
        }
        if (G == 4)
            hipLaunchKernelGGL((k_attn_pvd<HD, 4, Q8>), dim3(n_kv, ns + rows), dim3(192), 0, ST(s), scores, vc, pos0p,
                               n_kv, max_seq, out, c8, warm);
        else
            hipLaunchKernelGGL((k_attn_pvd<HD, 2, Q8>), dim3(n_kv, ns + rows), dim3(192), 0, ST(s), scores, vc, pos0p,
                               n_kv, max_seq, out, c8, warm);
    }
    else if (gm == 2)
        hipLaunchKernelGGL((k_attn_pvw<HD, 2, Q8>), dim3(n_kv, HD / 4), dim3(192), 0, ST(s), scores, vc, pos0p, n_q,
                           n_kv, max_seq, out, c8);
    else if (gm == 4)
        hipLaunchKernelGGL((k_attn_pvw<HD, 4, Q8>), dim3(n_kv, HD / 4), dim3(192), 0, ST(s), scores, vc, pos0p, n_q,
                           n_kv, max_seq, out, c8);
    else
        hipLaunchKernelGGL((k_attn_pvw<HD, 8, Q8>), dim3(n_kv, HD / 4), dim3(192), 0, ST(s), scores, vc, pos0p, n_q,
                           n_kv, max_seq, out, c8);
}

int32_t attn_wide_f32(void* s, int32_t lmax, const float* q, const float* kc, const float* vc, float* out,
                      float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                      float scale, const ScRope* rope, const DpufWarm* wm) {
    if (n_kv <= 0 || n_q % n_kv || (hd != 64 && hd != 128 && hd != 256)) return -1;
    if (lmax > max_seq) lmax = max_seq;
    const int G = n_q / n_kv;
    const int M = 1;
    // one-token decode with an even group: softmax once per row, then the
    // wide P.V (k_attn_pvd for groups of 2 and 4, else k_attn_pvw)
    {
        // chain segments of the softmax: 8 SEG positions per sum lane cover
        // keys up to 64 SEG
        const int segs[7] = {16, 32, 48, 64, 80, 96, 128};
        int seg = 0;
        for (int i = 0; i < 7 && !seg; i++)
            if (64 * segs[i] >= lmax) seg = segs[i];
        if (M == 1 && (G & 1) == 0 && G <= 8 && seg) {
            const int gm = G <= 2 ? 2 : G <= 4 ? 4 : 8;
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
#define WIDE_LAUNCH(HDV)                                                                                          \
    if (gm == 2) SC1_LAUNCH(HDV, 2) else if (gm == 4) SC1_LAUNCH(HDV, 4) else SC1_LAUNCH(HDV, 8)                  \
    smx_launch(s, seg, scores, pos0p, max_seq, n_q, n_kv, G, vc, HDV * 4);                                         \
    pv_wide_launch<HDV, false>(s, G, gm, scores, vc, pos0p, n_q, n_kv, max_seq, out, DpufKvQ8{}, wm);
            if (hd == 64) {
                WIDE_LAUNCH(64)
            } else if (hd == 128) {
                WIDE_LAUNCH(128)
            } else {
                WIDE_LAUNCH(256)
            }
#undef WIDE_LAUNCH
#undef SC1_LAUNCH
            LAUNCHED("k_attn_split_wide");
            attn_path_note(1);
            return 0;
        }
    }
    return -1;
}

int32_t attn_wide_q8(void* s, int32_t lmax, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd,
                     int32_t max_seq, float* scores, float* out, DpufKvQ8 c8, const DpufWarm* wm) {
    if (n_kv <= 0 || n_q % n_kv || (hd != 64 && hd != 128 && hd != 256)) return -1;
    if (lmax > max_seq) lmax = max_seq;
    const int G = n_q / n_kv;
    const int M = 1;
    // one token, groups of 2, 4, 6 or 8: the softmax once per row and the
    // wide P.V, as for the fp32 cache, with W = p * v_scale and V widened in
    // the producers
    if (M == 1 && (G & 1) == 0 && G <= 8) {
        const int segs[7] = {16, 32, 48, 64, 80, 96, 128};
        int seg = 0;
        for (int i = 0; i < 7 && !seg; i++)
            if (64 * segs[i] >= lmax) seg = segs[i];
        if (seg) {
            const int gm = G <= 2 ? 2 : G <= 4 ? 4 : 8;
            smx_launch(s, seg, scores, pos0, max_seq, n_q, n_kv, G, c8.vq, hd);
            if (hd == 64)
                pv_wide_launch<64, true>(s, G, gm, scores, nullptr, pos0, n_q, n_kv, max_seq, out, c8, wm);
            else if (hd == 128)
                pv_wide_launch<128, true>(s, G, gm, scores, nullptr, pos0, n_q, n_kv, max_seq, out, c8, wm);
            else
                pv_wide_launch<256, true>(s, G, gm, scores, nullptr, pos0, n_q, n_kv, max_seq, out, c8, wm);
            LAUNCHED("k_attn_q8_sc/k_attn_smx/wide P.V<q8>");
            return 0;
        }
    }
    return -1;
}
