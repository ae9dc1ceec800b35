// gemt.hip -- the few-token GEMM of the packed Mode 12 matrices (2 <= M <= 16
// rows of activations, K <= 4096): several sessions' decode steps in one pass
// over the weights (k_mvt), and its launch planning.
//
// Numerics contract: every output is the reference's per-row fp32 chain over
// the 32-column blocks in ascending order,
//   acc = fma(float(D - sum8), fp16(ws) * xs, acc)        (dpuf_avx2.c:2633-2635,
// the slab path dpuf_avx2.c:2643-2676), with D the u4 x i8 dot of the block and
// sum8 = 8 * sum(q): the same two rounded operations per block as k_gemm_mfma
// and k_gemm_skp, so the results are bit-identical to theirs.
//   * D - sum8 is an integer below 2^15 in magnitude: D exactly by one
//     v_mfma_i32_16x16x32_i8 per block (A = the nibbles u, 0..15 as int8,
//     B = the int8 activations), then an integer subtraction;
//   * fp16(ws) * xs is one v_fma_mix_f32 with a +0 addend (the product's
//     rounding; a zero product's sign cannot reach acc, which is never -0);
//   * build with -ffp-contract=off; fused multiply-adds are explicit fmaf.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <type_traits>

#include "hip_layer.h"
#include "dev_common.h"
#include "hip_internal.h"

// ---------------------------------------------------------------------------
// R waves compute a unit of P 16-row fragments (two 8-row groups each) for
// all M tokens, walking the blocks of K in order with the accumulators in
// registers.  MFMA D layout: lane l holds token column l % 16, rows
// 4 (l / 16) + v.  Each of the R waves repeats the unit's MFMAs and runs the
// chains of 4 / R of the four D components (R = 1 for large matrices, 2 or 4
// when the units alone would leave SIMDs idle).  No chain crosses a wave and
// no wave waits for another after the staging.
//
//   * 9..16 tokens (NT = 16 staged): P = 1, every D column is a token.
//   * up to 8 tokens (NT = 8): P = 2.  Lanes of columns 8..15 read token
//     l % 8, so each fragment's D repeats tokens 0..7 in both halves of every
//     16-lane row; one DPP move per register (row_shr:8, banks 2-3) puts
//     fragment b's columns 0..7 into columns 8..15 of fragment a's register,
//     so every lane of the chain instructions carries a distinct (row, token):
//     lane (i, kc) chains fragment i / 8, token i % 8.  Half the chain
//     instructions of two single-fragment waves, for one extra move each.
//
// A workgroup of MT_FW waves serves one job (matrix); it stages that job's
// activations once into LDS: the int8 values [block][token][32], so that an
// MFMA B fragment (lane l: token l % NT, columns 8 (l / 16) .. + 7 of the
// block) is one 8-byte read, and the block sums and scales [token][block]
// (four blocks in one read).
//
// Per unit a wave copies its groups' fp16 row scales (16 bytes per block) to
// an LDS area of its own, read per block.  The nibbles stream through a
// register ring PF 4-block quads deep: per quad and fragment one 16-byte
// buffer load per lane (lane offset fixed per unit, the quad in the scalar
// offset), row l % 16's bytes of block b0 + l / 16; a 4 x 4 transpose across
// the wave's 16-lane rows gives lane (i, kc) column chunk kc of all four
// blocks, the MFMA A layout.
// ---------------------------------------------------------------------------
#define MT_FW 4  // waves per workgroup
#define MT_RSRC3 0x00020000  // buffer descriptor word 3 (gfx9 family): 32-bit raw data

typedef int mt_i4 __attribute__((ext_vector_type(4)));

struct MtJob {
    const uint8_t* g;  // dense groups of the matrix (row-block layout)
    int g0, g1;        // groups computed
    int rows;
    const int8_t* q;   // activations int8 [M][K]
    const float* s;    // block scales [M][K/32]
    const int32_t* m;  // 8 * block sums [M][K/32]
    float* out;        // out[m * ldo + row]
    int ldo;
};

struct MtArgs {
    MtJob j[3];
    int n_jobs;
    int wb[4];  // prefix sums of the workgroups given to each job
    int K, M;
    // k_mvt<8, 1, 2, true>: a unit pairs 16 rows of gate (j[0]) with the same
    // rows of up (j[1]); the SwiGLU + prep of the down input [M][swI] goes to
    // swo (sign bits swsign, dead zone swdz)
    DpufPrep swo;
    const uint8_t* swsign;
    float swdz;
    int swI;
};

// LDS bytes of a workgroup: the staged activations of NT tokens (40 bytes
// per token and block) and each wave's copy of 2 P groups' row scales, every
// array with 4 blocks of padding (the reads one quad ahead run into it after
// the last quad; the scale rows of different tokens start on different banks).
static constexpr size_t mt_lds(int n_blk, int nt, int p) {
    return (size_t)(n_blk + 4) * ((nt + (p == 2)) * 32 + nt * 8 + MT_FW * 32 * p);
}

template <int NT, int R, int P, bool SWI = false>
__global__ __launch_bounds__(64 * MT_FW) void k_mvt(MtArgs A) {
    static_assert(P == 1 || NT == 8, "fragment pairs share the lanes of 8 staged tokens");
    static_assert(!SWI || (NT == 8 && R == 1 && P == 2), "the SwiGLU pairing: gate and up fragments, one wave each");
    constexpr int NV = 4 / R;            // D components per wave
    constexpr int FPW = MT_FW / R;       // units per workgroup round
    constexpr int PF = R == 1 || P == 2 ? 8 : 12;  // quads of nibbles in flight (even)
    constexpr int NG = 2 * P;            // groups per unit
    extern __shared__ __align__(16) uint8_t smem[];
    const int bid = blockIdx.x;
    int ji = 0;
    if (A.n_jobs > 1 && bid >= A.wb[1]) ji = 1;
    if (A.n_jobs > 2 && bid >= A.wb[2]) ji = 2;
    const MtJob& J = A.j[ji];
    const int K = A.K, M = A.M, n_blk = K >> 5, nq = n_blk >> 2;
    const int tid = threadIdx.x, l = tid & 63, i16 = l & 15, kc = l >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the descriptors stay scalar
    // unit slot; the wave's rows rotation rho: MFMA row 4c + k holds the
    // fragment's row 4c + ((k + rho) & 3), so D components 0 .. NV - 1 are
    // the fragment's rows 4c + rho + k, the ones this wave chains
    const int fs = w / R, rho = (w % R) * NV;
    // units of the job (SWI: 16 rows of gate and up, two groups of each)
    const int nun = SWI ? (J.g1 - J.g0) / 2 : (J.g1 - J.g0 + NG - 1) / NG;
    const int lb = bid - A.wb[ji], nwg = A.wb[ji + 1] - A.wb[ji];
    const uint32_t gstride = (uint32_t)n_blk * 144u;

    constexpr int NTS = NT + (P == 2);  // token slots per staged block (pairs: + a zero slot)
    const int nbp = n_blk + 4;  // padded block count of every LDS array
    int8_t* sq = (int8_t*)smem;                                       // [nbp][NTS][32]
    int32_t* sm = (int32_t*)(smem + (size_t)nbp * NTS * 32);          // sum8 [NT][nbp]
    float* sx = (float*)(smem + (size_t)nbp * (NTS * 32 + NT * 4));   // xs [NT][nbp]
    uint8_t* ws = smem + (size_t)nbp * (NTS * 32 + NT * 8) + (size_t)w * nbp * 16 * NG;  // [NG][nbp][16 B]

    // a unit's nibble loads: lane row i16 is row ri of fragment x (group
    // gf + 2 x + ri / 8, clamped into the job: a missing group repeats the
    // job's last, never stored), from one descriptor at group gf
    __amdgpu_buffer_rsrc_t rsc, rsb;  // SWI: rsc the gate groups of the unit, rsb the up groups
    uint32_t won[P];
    int ngr = NG;
    auto frag_setup = [&](int u) {
        const int ri = (i16 & 12) + ((i16 + rho) & 3);
        if constexpr (SWI) {
            const int gf = J.g0 + 2 * u;
            ngr = NG;
            rsc = __builtin_amdgcn_make_buffer_rsrc((void*)(A.j[0].g + (size_t)gf * gstride), 0, (int)(2 * gstride),
                                                    MT_RSRC3);
            rsb = __builtin_amdgcn_make_buffer_rsrc((void*)(A.j[1].g + (size_t)gf * gstride), 0, (int)(2 * gstride),
                                                    MT_RSRC3);
#pragma unroll
            for (int x = 0; x < P; x++)
                won[x] = (uint32_t)(ri >> 3) * gstride + (uint32_t)n_blk * 16u + (uint32_t)(ri & 7) * 16u +
                         (uint32_t)kc * 128u;
        } else {
            const int gf = J.g0 + NG * u;
            ngr = J.g1 - gf < NG ? J.g1 - gf : NG;
            rsc = __builtin_amdgcn_make_buffer_rsrc((void*)(J.g + (size_t)gf * gstride), 0, (int)(ngr * gstride),
                                                    MT_RSRC3);
#pragma unroll
            for (int x = 0; x < P; x++) {
                const int ga = min(gf + 2 * x + (ri >> 3), J.g1 - 1);
                won[x] = (uint32_t)(ga - gf) * gstride + (uint32_t)n_blk * 16u + (uint32_t)(ri & 7) * 16u +
                         (uint32_t)kc * 128u;
            }
        }
    };
    u32x4 wr[P][PF];
    auto quad_load = [&](int p, int qd) {
#pragma unroll
        for (int x = 0; x < P; x++)
            wr[x][p] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(SWI && x ? rsb : rsc, won[x], qd * 512, 0));
    };
    // the unit's row scales for this wave's LDS area: entry e = group
    // e / n_blk, block e % n_blk (NG n_blk <= 128 NG entries, 2 NG per lane),
    // loaded before the unit's first nibble quads so that the stores wait for
    // these loads only
    u32x4 st[2 * NG];
    auto scales_load = [&]() {
#pragma unroll
        for (int k = 0; k < 2 * NG; k++) {
            if constexpr (SWI) {
                // 64 | n_blk: entry l + 64 k lies in group (64 k) / n_blk for
                // every lane, so each load's descriptor is uniform
                const int gi = (64 * k) / n_blk, e = (64 * k) % n_blk + l;
                st[k] = __builtin_bit_cast(
                    u32x4, __builtin_amdgcn_raw_buffer_load_b128(gi >= 2 ? rsb : rsc,
                                                                  (uint32_t)(gi & 1) * gstride + (uint32_t)e * 16u, 0, 0));
            } else {
                const int e = min(l + 64 * k, NG * n_blk - 1), gi = min(e / n_blk, ngr - 1);
                st[k] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rsc, (uint32_t)gi * gstride + (uint32_t)(e % n_blk) * 16u, 0, 0));
            }
        }
    };
    auto scales_store = [&]() {
#pragma unroll
        for (int k = 0; k < 2 * NG; k++)
            if (l + 64 * k < NG * n_blk) {
                const int e = l + 64 * k;
                *(u32x4*)(ws + (size_t)((e / n_blk) * nbp + e % n_blk) * 16) = st[k];
            }
    };
    auto frag_start = [&](int u) {
        frag_setup(u);
        scales_load();
#pragma unroll
        for (int p = 0; p < PF; p++) quad_load(p, min(p, nq - 1));
    };
    int f = lb * FPW + fs;

    // staging through registers: every staging load, the stores, then the
    // first unit's loads (issued before them, the unit's loads delay the
    // staging data that every wave waits for); n_blk <= 128, chunk i of the
    // int8 rows = 16 bytes of (block i / 2 NT, token (i / 2) % NT, half i % 2)
    constexpr int QPT = 128 * NT * 2 / (64 * MT_FW), SPT = 128 * NT / (64 * MT_FW);
    mt_i4 tq[QPT];  // a native vector: an int4 struct array would stay in scratch
    int tm[SPT];
    float ts[SPT];
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int i = min(tid + 64 * MT_FW * k, n_blk * NT * 2 - 1);
        const int b = i / (2 * NT), t = (i >> 1) % NT, h = i & 1, tt = min(t, M - 1);
        tq[k] = *(const mt_i4*)(J.q + (size_t)tt * K + b * 32 + 16 * h);
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int i = min(tid + 64 * MT_FW * k, n_blk * NT - 1), b = i / NT, tt = min(i % NT, M - 1);
        tm[k] = J.m[(size_t)tt * n_blk + b];
        ts[k] = J.s[(size_t)tt * n_blk + b];
    }
#pragma unroll
    for (int k = 0; k < QPT; k++) {
        const int i = tid + 64 * MT_FW * k;
        if (i < n_blk * NT * 2) {
            const int b = i / (2 * NT), t = (i >> 1) % NT, h = i & 1;
            *(mt_i4*)(sq + (size_t)((b * NTS + t) * 2 + h) * 16) = tq[k];
        }
    }
    if (P == 2) {
        // each block's zero slot (the B columns that pair with the other fragment)
        for (int i = tid; i < nbp * 2; i += 64 * MT_FW)
            *(mt_i4*)(sq + (size_t)(((i >> 1) * NTS + NT) * 2 + (i & 1)) * 16) = (mt_i4){0, 0, 0, 0};
    }
#pragma unroll
    for (int k = 0; k < SPT; k++) {
        const int i = tid + 64 * MT_FW * k;
        if (i < n_blk * NT) {
            sm[(i % NT) * nbp + i / NT] = tm[k];
            sx[(i % NT) * nbp + i / NT] = ts[k];
        }
    }
    // (unconditional, clamped to the job's last unit when this slot has
    // none: the same loads on every path keep the later waits exact)
    frag_start(min(f, nun - 1));
    __syncthreads();

    const int tok = i16 % NT;
    const int fx = P == 2 ? i16 >> 3 : 0;  // the fragment this lane chains
    // B fragment of a block: P = 1, 8 bytes (token l % 16, columns 8 kc ..);
    // P = 2, 16 bytes, columns 16 (kc & 1) .. + 15 of token i16 % 8 when the
    // lane's column half (i16 / 8) matches its k half (kc / 2), else zeros
    const int8_t* sqt = P == 2 ? sq + ((i16 >> 3) == (kc >> 1) ? tok : NT) * 32 + (kc & 1) * 16
                               : sq + tok * 32 + kc * 8;
    const int32_t* smt = sm + tok * nbp;
    const float* sxt = sx + tok * nbp;
    for (; f < nun; f += nwg * FPW) {
        if (f != lb * FPW + fs) frag_start(f);
        // SWI: the down input's sign bits of this lane's 4 columns
        // 16 (f & 3) + 4 kc + k of block f / 4, loaded ahead of the K walk
        uint32_t sgn = 0;
        if constexpr (SWI)
            if (A.swsign) sgn = (uint32_t)(A.swsign[8 * (f >> 2) + 2 * (f & 3) + (kc >> 1)] >> (4 * (kc & 1))) & 0xFu;
        scales_store();
        // this lane's scales in the wave's copy: group 2 fx + kc / 2
        // (clamped), rows 4 (kc & 1) + rho .. of each block's 8
        const uint8_t* wst = ws + (size_t)min(2 * fx + (kc >> 1), ngr - 1) * nbp * 16 + (kc & 1) * 8 + rho * 2;
        float acc[NV];
#pragma unroll
        for (int v = 0; v < NV; v++) acc[v] = 0.0f;
        // LDS operands of a quad in slot sl: B fragments, the lane's row
        // scales (fp16 rows 4 (kc & 1) + rho + k, k < NV), and the four
        // blocks' token scales and sums; read one quad ahead of their use
        using BT = typename std::conditional<P == 2, mt_i4, long>::type;
        BT bb[2][4];
        uint32_t sw[2][4][2];
        float4 xq[2];
        int4 mq[2];
        auto lds_quad = [&](int sl, const int8_t* sqb, const int32_t* smb, const uint8_t* wsb, const float* sxb) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                bb[sl][j] = *(const BT*)(sqb + j * NTS * 32);
                if (NV == 4) {
                    const uint2 u = *(const uint2*)(wsb + j * 16);
                    sw[sl][j][0] = u.x;
                    sw[sl][j][1] = u.y;
                } else if (NV == 2) {
                    sw[sl][j][0] = *(const uint32_t*)(wsb + j * 16);
                } else {
                    sw[sl][j][0] = *(const uint16_t*)(wsb + j * 16);
                }
            }
            xq[sl] = *(const float4*)sxb;
            mq[sl] = *(const int4*)smb;
        };
        // one quad in ring slot p: its LDS operands were read a quad ahead
        // (slot p & 1), the next quad's are read now (after the last quad:
        // padding, never used); with `load`, the quad PF ahead (clamped to
        // the last) goes into the slot
        auto quad_step = [&](auto load, int p, int qd, const int8_t* sq0, const int32_t* sm0, const float* sx0,
                             const uint8_t* ws0) {
            const int cs = p & 1;  // PF is even: the slots alternate across rounds too
            lds_quad(cs ^ 1, sq0 + (4 * p + 4) * NTS * 32, sm0 + 4 * p + 4, ws0 + (4 * p + 4) * 16, sx0 + 4 * p + 4);
            const float xsj[4] = {xq[cs].x, xq[cs].y, xq[cs].z, xq[cs].w};
            const int xmj[4] = {mq[cs].x, mq[cs].y, mq[cs].z, mq[cs].w};
            mt_i4 dq[4];
            if constexpr (P == 2) {
                // lane row g held block g's 16 bytes of fragment a (x = 0)
                // and b; afterwards, per block j, rows 0-1 hold fragment a's
                // nibble words (0, 1) and (2, 3), rows 2-3 fragment b's
                uint32_t xa[4], ya[4];
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const auto t = __builtin_amdgcn_permlane32_swap(wr[0][p][r], wr[1][p][r], false, false);
                    xa[r] = t[0];  // rows: a blk 0, a blk 1, b blk 0, b blk 1
                    ya[r] = t[1];  // rows: a blk 2, a blk 3, b blk 2, b blk 3
                }
                const auto c0 = __builtin_amdgcn_permlane16_swap(xa[0], xa[2], false, false);
                const auto c1 = __builtin_amdgcn_permlane16_swap(xa[1], xa[3], false, false);
                const auto c2 = __builtin_amdgcn_permlane16_swap(ya[0], ya[2], false, false);
                const auto c3 = __builtin_amdgcn_permlane16_swap(ya[1], ya[3], false, false);
                const uint32_t pk[4][2] = {{c0[0], c1[0]}, {c0[1], c1[1]}, {c2[0], c3[0]}, {c2[1], c3[1]}};
                if constexpr (decltype(load)::value) quad_load(p, min(qd + PF, nq - 1));
                // one MFMA per block for both fragments: A rows = the 16
                // lane rows' fragment rows, k < 32 fragment a's block, k >= 32
                // fragment b's; B columns 0-7 carry the tokens at k < 32,
                // columns 8-15 at k >= 32, so D columns 8-15 are fragment b's
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const mt_i4 a = {(int)(pk[j][0] & 0x0F0F0F0Fu), (int)((pk[j][0] >> 4) & 0x0F0F0F0Fu),
                                     (int)(pk[j][1] & 0x0F0F0F0Fu), (int)((pk[j][1] >> 4) & 0x0F0F0F0Fu)};
                    dq[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, bb[cs][j], (mt_i4){0, 0, 0, 0}, 0, 0, 0);
                }
            } else {
                uint32_t w0 = wr[0][p][0], w1 = wr[0][p][1], w2 = wr[0][p][2], w3 = wr[0][p][3];
                skp_transpose(w0, w1, w2, w3);
                const uint32_t wj[4] = {w0, w1, w2, w3};
                if constexpr (decltype(load)::value) quad_load(p, min(qd + PF, nq - 1));
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const uint32_t lo = wj[j] & 0x0F0F0F0Fu, hi = (wj[j] >> 4) & 0x0F0F0F0Fu;
                    const long a = (long)(((uint64_t)hi << 32) | lo);
                    dq[j] = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bb[cs][j], (mt_i4){0, 0, 0, 0}, 0, 0, 0);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
#pragma unroll
                for (int k = 0; k < NV; k++) {
                    const gm_h2 h = __builtin_bit_cast(gm_h2, sw[cs][j][k >> 1]);
                    const float sp = __builtin_fmaf((float)h[k & 1], xsj[j], 0.0f);
                    acc[k] = fmaf((float)(dq[j][k] - xmj[j]), sp, acc[k]);
                }
            }
        };
        lds_quad(0, sqt, smt, wst, sxt);
        // rounds of PF quads that refill the ring, then the last round, which
        // loads nothing (no load of the wave outlives its unit)
        int q0 = 0;
        for (; q0 + PF < nq; q0 += PF) {
#pragma unroll
            for (int p = 0; p < PF; p++)
                quad_step(std::true_type{}, p, q0 + p, sqt + q0 * 4 * NTS * 32, smt + 4 * q0, sxt + 4 * q0,
                          wst + q0 * 64);
        }
#pragma unroll
        for (int p = 0; p < PF; p++) {
            // (a guard, not a break: a loop with an early exit is not unrolled)
            if (q0 + p < nq)  // uniform
                quad_step(std::false_type{}, p, q0 + p, sqt + q0 * 4 * NTS * 32, smt + 4 * q0, sxt + 4 * q0,
                          wst + q0 * 64);
        }
        if constexpr (SWI) {
            // lane i16 < 8: gate of token tok, rows 16 f + 4 kc + k; lane
            // i16 + 8 (row_ror 8): up of the same.  The workgroup's 4 units of
            // a round are the 64 columns of block f / 4 of the down input:
            // swiglu1 into LDS, then a 16-lane row per token preps the block
            // as swiglu_prep_lane does.
            float* yl = (float*)(smem + mt_lds(n_blk, NT, P));  // [NT][68]
            const int b64 = f >> 2;
#pragma unroll
            for (int k = 0; k < NV; k++) {
                const float up = DPP_F(acc[k], 0x128);
                const int c = 16 * (f & 3) + 4 * kc + k;
                if (i16 < 8) yl[tok * 68 + c] = swiglu1(acc[k], up, A.swdz, (sgn >> k) & 1u);
            }
            __syncthreads();
            if (tid < 16 * NT) {
                const int t = tid >> 4, r = tid & 15, I = A.swI, nbI = I >> 5;
                if (t < M) {  // uniform over the 16-lane row
                    float v4[4];
#pragma unroll
                    for (int k = 0; k < 4; k++) v4[k] = yl[t * 68 + 4 * r + k];
                    row_prep64(v4, r, b64, A.swo.q + (size_t)t * I, A.swo.s + (size_t)t * nbI,
                               A.swo.m + (size_t)t * nbI, A.swo.h ? A.swo.h + (size_t)t * I : nullptr);
                }
            }
            __syncthreads();
            continue;
        }
        // token tok of fragment fx, rows 4 (kc & 1) + rho + k of group
        // gf + 2 fx + kc / 2
        const int grp = J.g0 + NG * f + 2 * fx + (kc >> 1);
        if (tok < M && (P == 2 || i16 < NT) && grp < J.g1) {
#pragma unroll
            for (int k = 0; k < NV; k++) {
                const int r = grp * 8 + 4 * (kc & 1) + rho + k;
                if (r < J.rows) J.out[(size_t)tok * J.ldo + r] = acc[k];
            }
        }
    }
}

// ---------------------------------------------------------------------------

extern "C" {

typedef void (*MtKernel)(MtArgs);

// Workgroups of instance k the device holds at once with lds bytes each.
static int mt_capacity(MtKernel k, size_t lds) {
    static MtKernel c_k[8];
    static size_t c_lds[8];
    static int c_cap[8], c_n = 0;
    for (int i = 0; i < c_n; i++)
        if (c_k[i] == k && c_lds[i] == lds) return c_cap[i];
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, 64 * MT_FW, lds) != hipSuccess || per_cu <= 0)
        per_cu = 1;
    const int cap = per_cu * dpuf_hip_cu_count();
    if (c_n < 8) {
        c_k[c_n] = k;
        c_lds[c_n] = lds;
        c_cap[c_n++] = cap;
    }
    return cap;
}

int32_t dpuf_hip_mvt_launch(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs) {
    if (M < 2 || M > 16 || n_jobs < 1 || n_jobs > 3) return -1;
    const int K = jobs[0].w.cols, n_blk = K >> 5;
    if (K <= 0 || K % 128 || n_blk > 128) return -1;
    for (int i = 0; i < n_jobs; i++) {
        if (jobs[i].w.mode != 12 || jobs[i].w.cols != K || !jobs[i].p.q || !jobs[i].p.s || !jobs[i].p.m) return -1;
    }
    // up to 8 tokens: fragment pairs on 8 staged tokens; 9..16: single fragments
    const int nt = M <= 8 ? 8 : 16, pu = M <= 8 ? 2 : 1;
    int nun[3] = {0, 0, 0}, ftot = 0, utot = 0;
    for (int i = 0; i < n_jobs; i++) {
        const int ng = jobs[i].g1 - jobs[i].g0;
        ftot += ng > 0 ? (ng + 1) / 2 : 0;
        nun[i] = ng > 0 ? (ng + 2 * pu - 1) / (2 * pu) : 0;
        utot += nun[i];
    }
    if (ftot == 0) return 0;
    // up to one fragment per CU the K-split GEMM is faster (its workgroups
    // share a fragment's blocks instead of each walking all of K)
    if (ftot <= dpuf_hip_cu_count()) return -1;
    // waves per unit: as many as keep about two waves per SIMD busy (one for
    // pairs, whose waves carry twice the chains)
    const int target = (pu == 2 ? 4 : 8) * dpuf_hip_cu_count();
    const int R = 4 * utot <= target ? 4 : 2 * utot <= target ? 2 : 1;
    MtKernel k = pu == 2 ? (R == 4 ? k_mvt<8, 4, 2> : R == 2 ? k_mvt<8, 2, 2> : k_mvt<8, 1, 2>)
                         : (R == 4 ? k_mvt<16, 4, 1> : R == 2 ? k_mvt<16, 2, 1> : k_mvt<16, 1, 1>);
    const size_t lds = mt_lds(n_blk, nt, pu);
    int cap = mt_capacity(k, lds);
    if (dpuf_hip_mv_max_wg() > 0 && cap > dpuf_hip_mv_max_wg()) cap = dpuf_hip_mv_max_wg();
    MtArgs A;
    memset(&A, 0, sizeof A);
    A.n_jobs = n_jobs;
    A.K = K;
    A.M = M;
    for (int i = 0; i < n_jobs; i++) {
        A.j[i].g = jobs[i].w.g;
        A.j[i].g0 = jobs[i].g0;
        A.j[i].g1 = jobs[i].g1;
        A.j[i].rows = jobs[i].w.rows;
        A.j[i].q = jobs[i].p.q;
        A.j[i].s = jobs[i].p.s;
        A.j[i].m = jobs[i].p.m;
        A.j[i].out = jobs[i].out;
        A.j[i].ldo = jobs[i].ldo;
    }
    // each job's workgroups in proportion to its units, all resident at
    // once; a workgroup takes MT_FW / R units per round
    const int fpw = MT_FW / R;
    int wgs = 0;
    A.wb[0] = 0;
    for (int i = 0; i < n_jobs; i++) {
        const int need = (nun[i] + fpw - 1) / fpw;
        int nw = (int)(((long long)cap * nun[i] + utot - 1) / utot);
        nw = nw < 1 ? 1 : nw;
        wgs += nun[i] > 0 ? (nw < need ? nw : need) : 0;
        A.wb[i + 1] = wgs;
    }
    hipLaunchKernelGGL(k, dim3(wgs), dim3(64 * MT_FW), lds, ST(s), A);
    LAUNCHED("k_mvt");
    return 0;
}

// gate and up of 2 .. 8 tokens with the SwiGLU + prep of the down input in
// the same launch: a unit is 16 rows of gate and the same 16 of up, a
// workgroup round the 4 units of one 64-block of the down input.
int32_t dpuf_hip_mvt_swiglu(void* s, int32_t M, const DpufGemvJob* jobs, float dz, const uint8_t* sign,
                            DpufPrep out) {
    const DpufGemvJob& a = jobs[0];
    const DpufGemvJob& b = jobs[1];
    const int K = a.w.cols, I = a.w.rows, n_blk = K >> 5;
    if (M < 2 || M > 8 || a.w.mode != 12 || b.w.mode != 12 || b.w.cols != K || b.w.rows != I || K <= 0 ||
        K % 2048 || n_blk > 128 || I <= 0 || I % 64 || a.g0 != 0 || b.g0 != 0 || a.g1 != I / 8 || b.g1 != I / 8 ||
        !a.p.q || !a.p.s || !a.p.m || a.p.q != b.p.q || a.p.s != b.p.s || a.p.m != b.p.m || !out.q || !out.s ||
        !out.m || out.q == a.p.q)
        return -1;
    // one wave per unit (the pairing's layout): taken where the plain launch
    // would also run one wave per unit pair, i.e. units > 2 per CU
    const int nun = I / 16;
    if (nun <= 2 * dpuf_hip_cu_count()) return -1;
    MtKernel k = k_mvt<8, 1, 2, true>;
    const size_t lds = mt_lds(n_blk, 8, 2) + 8 * 68 * sizeof(float);
    int cap = mt_capacity(k, lds);
    if (dpuf_hip_mv_max_wg() > 0 && cap > dpuf_hip_mv_max_wg()) cap = dpuf_hip_mv_max_wg();
    MtArgs A;
    memset(&A, 0, sizeof A);
    A.n_jobs = 1;
    A.K = K;
    A.M = M;
    for (int i = 0; i < 2; i++) {
        A.j[i].g = jobs[i].w.g;
        A.j[i].g0 = 0;
        A.j[i].g1 = I / 8;
        A.j[i].rows = I;
        A.j[i].q = a.p.q;
        A.j[i].s = a.p.s;
        A.j[i].m = a.p.m;
    }
    A.swo = out;
    A.swsign = sign;
    A.swdz = dz;
    A.swI = I;
    const int need = nun / MT_FW;  // every workgroup takes whole rounds of MT_FW units
    const int wgs = cap < need ? cap : need;
    A.wb[0] = 0;
    A.wb[1] = wgs;
    hipLaunchKernelGGL(k, dim3(wgs), dim3(64 * MT_FW), lds, ST(s), A);
    LAUNCHED("k_mvt");
    return 0;
}

}  // extern "C"
