// gemm.hip -- the M > 1 GEMM of the packed matrices: the MFMA slab GEMM
// (k_gemm_mfma) and the K-split GEMMs for up to 16 rows (k_gemm_sk,
// k_gemm_skp), with their launch planning.
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
// A workgroup of NW = 4 or 8 waves computes 16 NW GM_RF rows x 16 TT tokens;
// wave w owns GM_RF 16-row fragments and all the tokens as TT 16-token tiles
// (GM_RF TT MFMAs per block).  With 8 waves twice the rows share a staged
// token tile: half the activation staging per MFMA.  Activations arrive as fp16 (DpufPrep.h, written by the
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
// Launches of at least this many rows (the fused gate + up projection) and
// more than GM_NW8_MINM tokens take 8-wave workgroups: pp512 at the 8B shape
// 21.2 -> 20.85 ms, pp256 13.2 -> 13.0 ms, pp128 10.2 -> 10.5 ms (half the
// workgroups of the 4-wave grid leave CUs idle), pp32 and pp64 unchanged;
// Q/K/V, O and down on 8 waves as well, pp512 21.1 ms; down as well, 20.8 ms.
#define GM_NW8_ROWS 16384
#define GM_NW8_MINM 128

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
    int32_t* err;  // device error word: set when a bounded wait of k_gemm_sk runs out
    // gate + up with the SwiGLU (k_gemm_mfma<..., true>): the prep of the
    // down projection's input [M][swI] goes to swo, with the down input's
    // sign bits swsign and dead zone swdz
    DpufPrep swo;
    const uint8_t* swsign;
    float swdz;
    int swI;
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
template <int TT, int RF, int MODE, int NW, bool SWI = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(MODE == 12 ? 4 : 2))) void k_gemm_mfma(
    GmArgs A) {
    constexpr int NT = 16 * TT;  // tokens per workgroup
    constexpr int NTH = 64 * NW;  // threads per workgroup
    constexpr int GPW = 2 * RF * NW;  // 8-row groups per workgroup
    constexpr bool ASYM = MODE != 12;
    static_assert(GM_SB % 2 == 0, "a stage holds whole 64-blocks");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(!SWI || (NW == 8 && RF == 1 && TT == 4 && MODE == 12), "the SwiGLU pairing: 4 + 4 waves");
    __shared__ __align__(16) uint8_t bq[2][GM_SB][NT][64];  // f16 activations [stage][block][token][k]
    __shared__ __align__(16) float bs[2][GM_SB][16][TT];    // block scales [stage][block][token % 16][token / 16]
    __shared__ __align__(16) int32_t bm[ASYM ? 2 : 1][GM_SB][16][TT];  // 8 * block sums (modes 13 / 14)
    __shared__ __align__(16) uint32_t bw[2][GM_SB][4 * GPW];  // weight scales [stage][block][group * 4 + word]
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
            for (int t = threadIdx.x >> 6; t < 16 * TT; t += NW) {
                const int m = ty * 16 * TT + t;
                if (m < A.M && r < A.z1) A.zo[(size_t)m * A.zld + r] = 0.0f;
            }
        }
        return;
    }
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, i16 = l & 15, kc = l >> 4;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    // SWI: waves 0-3 compute job 0 (gate), waves 4-7 job 1 (up), the same 64
    // rows (8 groups) of each, and the activations are the jobs' shared input
    int ji = 0;
    if (SWI) {
        ji = wu >> 2;
    } else {
        if (A.n_jobs > 1 && rt >= A.tb[1]) ji = 1;
        if (A.n_jobs > 2 && rt >= A.tb[2]) ji = 2;
    }
    // the job's fields picked from the kernel arguments by uniform selects,
    // so they stay in scalar registers through the loop
    const GmJob& J = ji == 0 ? A.j[0] : ji == 1 ? A.j[1] : A.j[2];
    const uint16_t* const Jh = ji == 0 ? A.j[0].h : ji == 1 ? A.j[1].h : A.j[2].h;
    const float* const Js = ji == 0 ? A.j[0].s : ji == 1 ? A.j[1].s : A.j[2].s;
    const int32_t* const Jm = ji == 0 ? A.j[0].m : ji == 1 ? A.j[1].m : A.j[2].m;
    // first group of the workgroup (SWI: of the wave's job), and the wave's
    // place among the waves of that job
    const int gb = SWI ? J.g0 + rt * (GPW / 2) : J.g0 + (rt - A.tb[ji]) * GPW;
    const int wl = SWI ? (wu & 3) : wu;
    const int m0 = ty * NT;
    const int K = A.K, M = A.M, n_blk = K >> 5;
    const size_t gstride = (size_t)n_blk * (MODE == 14 ? 208 : 144);

    // Every load is a buffer load: a wave-uniform descriptor, a 32-bit lane
    // offset fixed for the launch and a scalar block offset, so addressing
    // costs no vector instructions in the loop (and a load past a
    // descriptor's range reads 0 instead of faulting).  Weights of the
    // wave's RF fragments (groups clamped into the job) are addressed from
    // the wave's first group.
    const int gw0 = min(gb + 2 * RF * wl, J.g1 - 1);
    const size_t wbytes = (size_t)(J.g1 - gw0) * gstride;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(J.g + (size_t)gw0 * gstride), 0, (int)(wbytes < 0xFFFFFFFFu ? wbytes : 0xFFFFFFFFu), GM_RSRC3);
    uint32_t on[RF], oh[RF];
#pragma unroll
    for (int f = 0; f < RF; f++) {
        const int ga = min(gb + 2 * RF * wl + 2 * f + (i16 >> 3), J.g1 - 1);
        on[f] = (uint32_t)((size_t)(ga - gw0) * gstride + (size_t)n_blk * 16 + (i16 & 7) * 16 + kc * 4);
        // mode 14: the lane's high-bit word (chunk kc's bits are in word kc / 2)
        oh[f] = (uint32_t)((size_t)(ga - gw0) * gstride + (size_t)n_blk * 144 + (i16 & 7) * 8 + (kc >> 1) * 4);
    }
    // Weight scales go through LDS with the activations: a stage's GPW
    // groups x GM_SB blocks x 8 fp16 scales are WD dwords, dword d = (tid +
    // NTH k) % WD (group d / (4 GM_SB), block (d / 4) % GM_SB, word d % 4),
    // addressed from the workgroup's first group; threads past WD repeat a
    // dword.  Blocks past the end read bytes that are never used.
    // SWI: groups 0-7 of a stage are job 0's, 8-15 job 1's; with one dword
    // per thread (d = tid % 256) a wave's dwords are all of one job.
    constexpr int WD = 4 * GPW * GM_SB, WPT = (WD + NTH - 1) / NTH;
    static_assert(!SWI || (WPT == 1 && WD == 256), "one job per wave's scale dwords");
    const int jg = SWI ? (wu & 3) >> 1 : ji;
    const GmJob& JG = jg == 0 ? A.j[0] : jg == 1 ? A.j[1] : A.j[2];
    const int gbg = SWI ? JG.g0 + rt * (GPW / 2) : gb;
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(JG.g + (size_t)gbg * gstride), 0,
        (int)((size_t)(JG.g1 - gbg) * gstride < 0xFFFFFFFFu ? (size_t)(JG.g1 - gbg) * gstride : 0xFFFFFFFFu),
        GM_RSRC3);
    uint32_t og[WPT], sw[WPT];  // load offsets; the thread's scale dwords of the stage in flight
    int wgi[WPT];               // their LDS word index in a stage buffer
#pragma unroll
    for (int k = 0; k < WPT; k++) {
        const int wd = (tid + NTH * k) % WD, g = wd / (4 * GM_SB), b = (wd >> 2) % GM_SB, w4 = wd & 3;
        const int gj = SWI ? (g & (GPW / 2 - 1)) : g;  // the group within its job's rows
        og[k] = (uint32_t)((size_t)(min(gbg + gj, JG.g1 - 1) - gbg) * gstride + b * 16 + w4 * 4);
        wgi[k] = b * 4 * GPW + g * 4 + w4;
    }
    // staging: a stage holds NT tokens x GM_SB blocks of 64 fp16 bytes, four
    // 16-byte chunks each.  Chunk c = tid + NTH k of the stage is chunk c & 3
    // of pair c / 4 = (token (c / 4) % NT, block (c / 4) / NT), so the 64
    // lanes of a load read 16 tokens' 64 contiguous bytes.  Scale i = tid +
    // NTH k is pair i.  Loads are unconditional, at token and block clamped
    // into range: a token past M only feeds output columns that are never
    // stored, a block past the end is never computed, and a load without a
    // branch around it keeps the compiler's wait counts exact.
    constexpr int CPT = NT * GM_SB * 4 / NTH, SPT = (NT * GM_SB + NTH - 1) / NTH;
    static_assert(CPT >= 1 && NT * GM_SB * 4 % NTH == 0, "whole chunks per thread");
    const int n_st = (n_blk + GM_SB - 1) / GM_SB;
    gm_u4 sq[CPT];  // a native vector: a struct copy would keep the array in scratch
    float ss[SPT];
    int32_t sm[SPT];
    // byte offsets of the token rows (M K < 2^30 is checked at launch); with
    // NT = 64 a chunk's block (wave / 4 + NW k / 4) and a scale's block (the
    // wave, + NW k) are uniform and go into the scalar offset
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc((void*)Jh, 0, M * K * 2, GM_RSRC3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)Js, 0, M * n_blk * 4, GM_RSRC3);
    const __amdgpu_buffer_rsrc_t rm =
        __builtin_amdgcn_make_buffer_rsrc(ASYM ? (void*)Jm : (void*)Js, 0, M * n_blk * 4, GM_RSRC3);
    uint32_t ho[CPT], so[SPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int pr = (tid >> 2) + (NTH / 4) * k, m = min(m0 + pr % NT, M - 1);
        const int sbt = NT == 64 ? 0 : pr / NT;
        ho[k] = (uint32_t)(2 * (m * K + 32 * sbt + 8 * (tid & 3)));
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int i = min(tid + NTH * k, NT * GM_SB - 1), m = min(m0 + i % NT, M - 1);
        const int sbt = NT == 64 ? 0 : i / NT;
        so[k] = (uint32_t)(4 * (m * n_blk + sbt));
    }
    // the stage's first block, clamped so that a stage's blocks stay in range
    // when it starts in range (blocks past the end are never computed)
    auto stage_load = [&](int st) {
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int sbt = NT == 64 ? (wu >> 2) + k * (NW / 4) : 0;
            const int b = NT == 64 ? min(st * GM_SB + sbt, n_blk - 1) : st * GM_SB;
            sq[k] = __builtin_bit_cast(gm_u4, __builtin_amdgcn_raw_buffer_load_b128(rh, ho[k], b * 64, 0));
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int b = NT == 64 ? min(st * GM_SB + wu + NW * k, n_blk - 1) : st * GM_SB;
            ss[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, so[k], b * 4, 0));
            if (ASYM) sm[k] = (int32_t)__builtin_amdgcn_raw_buffer_load_b32(rm, so[k], b * 4, 0);
        }
#pragma unroll
        for (int k = 0; k < WPT; k++) sw[k] = __builtin_amdgcn_raw_buffer_load_b32(rg, og[k], st * GM_SB * 16, 0);
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int k = 0; k < CPT; k++) {
            const int c = tid + NTH * k, pr = c >> 2, tk = pr % NT, sbt = pr / NT, qu = c & 3;
            *(gm_u4*)&bq[buf][sbt][tk][16 * (qu ^ ((tk >> 1) & 3))] = sq[k];
        }
#pragma unroll
        for (int k = 0; k < SPT; k++) {
            const int i = tid + NTH * k, tk = i % NT, sbt = i / NT;
            if (NT * GM_SB % NTH == 0 || i < NT * GM_SB) {
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

    if constexpr (SWI) {
        // SwiGLU + prep of the down input for the workgroup's 64 columns
        // (one 64-block, blk) of the M tokens m0 .. m0 + 63.  Lane l of wave
        // w holds acc[0][t][v] for column c = 16 (w & 3) + 4 (l / 16) + v and
        // token 16 t + l % 16; x[w & 3][t][v][l] in the LDS of the stage
        // buffers (free once every wave is past its last block) exchanges
        // them: the up waves write theirs, the gate waves replace them by
        // swiglu1(gate, up) (swiglu_prep_lane's arithmetic), then each 16-lane
        // row preps one token's block as swiglu_prep_lane does.
        float* x = (float*)&bq[0][0][0][0];
        static_assert(sizeof(bq) >= 4 * TT * 4 * 64 * sizeof(float), "the exchange fits the stage buffers");
        auto xi = [&](int ww, int t, int v, int ln) { return ((ww * TT + t) * 4 + v) * 64 + ln; };
        const int blk = (gb * 8) >> 6;  // gb: the wave's first group; a block is 8 groups
        __syncthreads();
        if (wu >= 4) {
#pragma unroll
            for (int t = 0; t < TT; t++)
#pragma unroll
                for (int v = 0; v < 4; v++) x[xi(wl, t, v, l)] = acc[0][t][v];
        }
        __syncthreads();
        if (wu < 4) {
            const uint8_t* sg = A.swsign ? A.swsign + 8 * blk : nullptr;
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int c = 16 * wl + 4 * kc + v;
                const uint32_t neg = sg ? (sg[c >> 3] >> (c & 7)) & 1u : 0u;
#pragma unroll
                for (int t = 0; t < TT; t++) x[xi(wl, t, v, l)] = swiglu1(acc[0][t][v], x[xi(wl, t, v, l)], A.swdz, neg);
            }
        }
        __syncthreads();
        const int R = tid >> 4, r = tid & 15, I = A.swI, nbI = I >> 5;
#pragma unroll
        for (int pass = 0; pass < NT / 32; pass++) {
            const int tok = R + 32 * pass, mt = m0 + tok;
            if (mt < M) {  // uniform over the 16-lane row
                float v4[4];
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const int c = 4 * r + k;
                    v4[k] = x[xi(c >> 4, tok >> 4, c & 3, 16 * ((c >> 2) & 3) + (tok & 15))];
                }
                row_prep64(v4, r, blk, A.swo.q + (size_t)mt * I, A.swo.s + (size_t)mt * nbI,
                           A.swo.m + (size_t)mt * nbI, A.swo.h ? A.swo.h + (size_t)mt * I : nullptr);
            }
        }
        return;
    }
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
#ifndef SK_NB
#define SK_NB 4   // k_gemm_sk round buffers in LDS (producers run up to SK_NB rounds ahead of the chains)
#endif

#define SKP_P 8  // ring depth in rounds: a multiple of every NR
#define SKP_RB 4                 // blocks per producer wave per round
#define SKP_RS (SK_NP * SKP_RB)  // 32 blocks per round

// One round of a chain wave: every block's sp = fp16(ws) * xs first (they
// do not depend on the chain), then acc = fma(d, sp, acc) over the round's
// blocks in order; a full round runs the chain with no per-block guard, so
// each block adds one dependent instruction, not three (product, fma and a
// select).
DEV float sk_round_chain(float acc, const float (&d)[SKP_RS], const uint32_t (&wv)[SKP_RS / 2],
                         const gm_f4 (&xr)[SKP_RS / 4], int nj) {
    float sp[SKP_RS];
#pragma unroll
    for (int j = 0; j < SKP_RS; j++) {
        const gm_h2 hw = __builtin_bit_cast(gm_h2, wv[j >> 1]);
        sp[j] = __builtin_fmaf((float)hw[j & 1], xr[j >> 2][j & 3], 0.0f);
    }
    if (nj >= SKP_RS) {
#pragma unroll
        for (int j = 0; j < SKP_RS; j++) acc = fmaf(d[j], sp[j], acc);
    } else {
#pragma unroll
        for (int j = 0; j < SKP_RS; j++)
            if (j < nj) acc = fmaf(d[j], sp[j], acc);
    }
    return acc;
}

// Polls an LDS counter until it reaches want, at most 2^22 polls (false when
// it ran out); the polled value is wave-uniform, so the loop is scalar.
DEV bool sk_wait(uint32_t* p, uint32_t want) {
    int spins = 0;
#pragma clang loop unroll(disable)
    while ((uint32_t)__builtin_amdgcn_readfirstlane(
               (int)__hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < want) {
        if (++spins >= (1 << 22)) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    return true;
}

__global__ __launch_bounds__(64 * (SK_NP + SK_NC)) void k_gemm_sk(GmArgs A) {
    __shared__ __align__(16) float dq[SK_NB][SKP_RS][4][64];    // D tiles [buf][block][v][lane]
    __shared__ __align__(16) uint16_t wsl[SK_NB][16][SKP_RS];   // weight scales [buf][row][block]
    __shared__ __align__(16) float xsl[SK_NB][16][SKP_RS + 4];  // token scales [buf][token][block], rows padded
    // hand-off counters per buffer, cumulative: full[b] counts producer waves
    // done with a round in b, freed[b] chain waves done reading one
    __shared__ uint32_t full[SK_NB], freed[SK_NB];
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
    if (tid < SK_NB) {
        full[tid] = 0;
        freed[tid] = 0;
    }
    __syncthreads();

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
        for (int it0 = 0; it0 < n_r; it0 += SK_P) {
#pragma unroll
            for (int u = 0; u < SK_P; u++) {
                const int it = it0 + u;
                if (it >= n_r) break;  // uniform
                const int un = (u + SK_P - 1) % SK_P;
                load(it + SK_P - 1, wq[un], wsq[un], ax[un], xsq[un]);
                {
                    // round it goes to buffer it % SK_NB once the chains have
                    // read round it - SK_NB from it
                    const int buf = it % SK_NB;
                    if (it >= SK_NB) {
                        if (!sk_wait(&freed[buf], (uint32_t)(SK_NC * (it / SK_NB))) && l == 0) atomicOr(A.err, 1);
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
                    }
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
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
                    if (l == 0) __hip_atomic_fetch_add(&full[buf], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
                }
            }
        }
        return;
    }

    // ---- chain wave c: output (token l % 16, row 4 (l / 16) + c) ----
    const int c = w - SK_NP, rr = 4 * kc + c;
    float acc = 0.0f;
    for (int it = 1; it <= n_r; it++) {
        {
            // round it - 1, once every producer wave has written it
            const int buf = (it - 1) % SK_NB, b0 = (it - 1) * SKP_RS;
            if (!sk_wait(&full[buf], (uint32_t)(SK_NP * ((it - 1) / SK_NB + 1))) && l == 0) atomicOr(A.err, 1);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
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
            acc = sk_round_chain(acc, d, wv, xr, nj);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
            if (l == 0) __hip_atomic_fetch_add(&freed[buf], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
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
                    acc = sk_round_chain(acc, d, wv, xr, nj);
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


extern "C" {

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


// Gate and up of M > 16 tokens with the SwiGLU + dead zone + prep of the down
// input in the same launch (k_gemm_mfma<..., true>): a workgroup's
// waves 0-3 compute 64 rows of gate, waves 4-7 the same 64 rows of up, from
// the activations both share, and the workgroup preps those 64 columns of
// every token into out.  -1 (nothing launched) when the shapes do not allow
// it: mode 12, one shared input, every row of equal gate / up matrices with
// 64 | rows, fp16 activations, and out distinct from the input.  Unlike the
// plain gate+up launch it pays at every M > 16 (pp32 8.7 -> 8.6 ms, pp64 9.3
// -> 9.1, pp128 10.2 either way, pp512 20.7 -> 19.8 at the 8B shape).
int32_t dpuf_hip_gemm_swiglu(void* s, int32_t M, const DpufGemvJob* jobs, float dz, const uint8_t* sign,
                             DpufPrep out) {
    const DpufGemvJob& a = jobs[0];
    const DpufGemvJob& b = jobs[1];
    const int I = a.w.rows;
    if (M <= 16 || a.w.mode != 12 || b.w.mode != 12 || a.w.cols != b.w.cols || b.w.rows != I || I % 64 ||
        2 * I < GM_NW8_ROWS || a.g0 != 0 || b.g0 != 0 || a.g1 != I / 8 || b.g1 != I / 8 || !a.p.h || a.p.h != b.p.h ||
        a.p.s != b.p.s || !out.q || !out.s || !out.m || !out.h || out.h == a.p.h || out.q == a.p.q)
        return -1;
    if ((long long)M * a.w.cols >= (1ll << 30) || (long long)M * I >= (1ll << 30)) return -1;
    GmArgs G;
    memset(&G, 0, sizeof G);
    G.n_jobs = 2;
    G.K = a.w.cols;
    G.M = M;
    for (int i = 0; i < 2; i++) {
        G.j[i].g = jobs[i].w.g;
        G.j[i].g0 = 0;
        G.j[i].g1 = jobs[i].g1;
        G.j[i].rows = jobs[i].w.rows;
        G.j[i].h = jobs[i].p.h;
        G.j[i].s = jobs[i].p.s;
        G.j[i].m = jobs[i].p.m;
        G.j[i].out = jobs[i].out;
        G.j[i].ldo = jobs[i].ldo;
    }
    const int tiles = I / 64;
    G.tb[0] = 0;
    G.tb[1] = tiles;
    G.tb[2] = tiles;
    G.swo = out;
    G.swsign = sign;
    G.swdz = dz;
    G.swI = I;
    const int gx = (tiles + 7) & ~7;
    G.gy = (M + 16 * GM_TT - 1) / (16 * GM_TT);
    const dim3 grid = GM_XCD ? dim3(gx * G.gy) : dim3(gx, G.gy);
    hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 12, 8, true>), grid, dim3(512), 0, ST(s), G);
    LAUNCHED("k_gemm_mfma");
    return 0;
}

// The M > 1 GEMM; rows [z0, z1) of zo are zeroed by the same launch.
void dpuf_hip_gm_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs, float* zo, int32_t zld, int32_t z0,
                      int32_t z1) {
    {
        GmArgs G;
        memset(&G, 0, sizeof G);
        int t = 0;
        // 8-wave workgroups (128 rows sharing one staged token tile) for the
        // launches with the most rows, 4-wave ones otherwise
        int rows_all = 0;
        for (int i = 0; i < n_jobs; i++) rows_all += jobs[i].g1 > jobs[i].g0 ? 8 * (jobs[i].g1 - jobs[i].g0) : 0;
        const int nw = jobs[0].w.mode == 12 && M > GM_NW8_MINM && rows_all >= GM_NW8_ROWS ? 8 : 4;
        const int gpw = 2 * GM_RF * nw;
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
            t += ng > 0 ? (ng + gpw - 1) / gpw : 0;
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
            if (dpuf_hip_mv_max_wg() > 0 && cap > dpuf_hip_mv_max_wg()) cap = dpuf_hip_mv_max_wg();
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
            G.err = dpuf_hip_error_word();
            if (!G.err) {
                note(hipErrorInvalidValue, "dpuf_hip_gemv: no device error word bound");
                return;
            }
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
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 13, 4>), grid, dim3(256), 0, ST(s), G);
        else if (mode == 14)
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 14, 4>), grid, dim3(256), 0, ST(s), G);
        else if (nw == 8)
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 12, 8>), grid, dim3(512), 0, ST(s), G);
        else
            hipLaunchKernelGGL((k_gemm_mfma<GM_TT, GM_RF, 12, 4>), grid, dim3(256), 0, ST(s), G);
        LAUNCHED("k_gemm_mfma");
    }
}


}  // extern "C"
