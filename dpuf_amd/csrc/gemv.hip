// gemv.hip -- the M == 1 GEMV of the packed Mode 12 / 13 / 14 matrices
// (k_mv) and its launch planning, the producer-fed launches, the cache
// warm-up plan, and the dispatch of dpuf_hip_gemv to the M > 1 GEMM.
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
    // LM-head reductions: when set, every chain (each chain wave, or wave 0
    // of a one-group workgroup) writes the partial of the rows it computed,
    // red[workgroup * chains per workgroup + chain] (not on a skipped launch)
    lm4* red;
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
DEV void mv_chains(const MvGeo& G, int c, int n_my, int lane, uint8_t* smem, MvSync* sy, lm4* red) {
    lm4 part = lm_part_init();
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
            if (r < G.rows) {
                G.out[r] = acc;
                if (red) part = lm_part_take(part, acc, r);
            }
        }
        __builtin_amdgcn_s_setprio(0);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
        if (lane == 0) __hip_atomic_store(&sy->done[buf], lg, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (red) {
        part = lm_part_wave(part);
        if (lane == 0) red[blockIdx.x * MV_NC + c] = part;
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
// copies take the step serial.  No agent-scope release fence precedes the
// flag stores: on gfx950 that fence is an L2 writeback walking the whole
// cache, and the data stores above already went through to memory and were
// acknowledged (vmcnt 0) before the barrier.  The consumers' ordinary loads
// of the data rely on the L1/L2 invalidate that the dispatch packet's
// acquire fence performs at the start of every launch, graph nodes included.
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
        mv_chains(G, w - G.NW, n_my, lane, smem, &sy, A.red);
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
        if (w == 0) {
            lm4 part = lm_part_init();
            if (lane < 8) {
                const float acc = run_chain<MV_CHAIN1>((const float4*)((float2*)smem + lane * G.ld), G.n_blk >> 1);
                const int r = G.g0 * 8 + G.lb * 8 + lane;
                if (r < G.rows) {
                    G.out[r] = acc;
                    if (A.red) part = lm_part_take(part, acc, r);
                }
            }
            if (A.red) {
                part = lm_part_wave(part);
                if (lane == 0) A.red[blockIdx.x] = part;
            }
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

extern "C" {

typedef void (*MvKernel)(MvArgs);

static int g_mv_max_wg = 0;  // test/tuning cap on GEMV / K-split GEMM workgroups


void dpuf_hip_set_gemv_max_wg(int32_t n) { g_mv_max_wg = n > 0 ? n : 0; }

// Device error word of the current API call on this thread (see MvArgs::err).
static thread_local int32_t* g_err_word = NULL;

void dpuf_hip_bind_error_word(int32_t* d_word) { g_err_word = d_word; }
int32_t* dpuf_hip_error_word(void) { return g_err_word; }

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

// One launch over jobs of one mode; returns the chains of the launch (the
// partials it writes when A.red is set), 0 when there is nothing to launch,
// -1 on an error (reported), including more chains than red_cap.
static int mv_launch(void* s, MvArgs& A, const int* n_groups, int mode, int red_cap = 0) {
    const int n_blk = A.K >> 5;
    MvKernel k, k1;
    int nw, most;
    if (mv_plan(A.n_jobs, n_groups, A.K, mode, k, k1, nw, A.wb, most) == 0) return 0;
    const int grid = A.wb[A.n_jobs];
    const size_t buf = (size_t)8 * (n_blk + 2) * 8;
    if (!g_err_word) {
        note(hipErrorInvalidValue, "dpuf_hip_gemv: no device error word bound");
        return -1;
    }
    A.err = g_err_word;
    A.nbuf = most < MV_NBUF ? most : MV_NBUF;
    A.nc = most > 1 ? MV_NC : 0;
    const int chains = grid * (A.nc ? MV_NC : 1);
    if (A.red && chains > red_cap) {
        note(hipErrorInvalidValue, "dpuf_hip_gemv_red: more partials than the buffer holds");
        return -1;
    }
    const int threads = (nw + A.nc) * 64;
    const size_t lds = (size_t)A.nbuf * buf;
    hipLaunchKernelGGL(A.nc ? k : k1, dim3(grid), dim3(threads), lds, ST(s), A);
    LAUNCHED("k_mv");
    return chains;
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
// The plan of a producer-fed launch of job over I activations: kernel,
// threads, producers, GEMV workgroups, LDS bytes; false when it does not apply.
static bool fed_plan(int32_t I, const DpufGemvJob* job, MvKernel& kf, int& threads, int& np, int& nwg, size_t& lds) {
    const int mode = job->w.mode;
    if ((mode != 12 && mode != 13 && mode != 14) || job->w.cols != I || I <= 0 || I % 64) return false;
    const int n_blk = I >> 5, S = (n_blk + 7) >> 3;
    if (S > (MV_HOIST48 ? 4 : 3) * (16 - MV_NC)) return false;  // activations loaded per round: no such mode
    const int ng = job->g1 - job->g0 > 0 ? job->g1 - job->g0 : 0;
    MvKernel k, k1;
    int nw, most, wb[4] = {0, 0, 0, 0};
    if (mv_plan(1, &ng, I, mode, k, k1, nw, wb, most) == 0 || most != 1) return false;
    threads = nw * 64;
    np = (I / 4 + threads - 1) / threads;
    if (np > 64) return false;
    const int nl = S <= 16 - MV_NC ? 1 : S <= 2 * (16 - MV_NC) ? 2 : S <= 3 * (16 - MV_NC) ? 3 : 4;
    kf = mv_fed_kernel(mode, nl);
    lds = (size_t)8 * (n_blk + 2) * 8;
    nwg = wb[1];
    return ng <= mv_capacity(kf, threads, lds);  // every GEMV workgroup resident at once
}

int32_t dpuf_hip_fed_producers(int32_t I, const DpufGemvJob* job) {
    MvKernel kf;
    int threads, np, nwg;
    size_t lds;
    return fed_plan(I, job, kf, threads, np, nwg, lds) ? np : 0;
}

int32_t dpuf_hip_swiglu_gemv(void* s, int32_t I, const float* gate, const float* up, float dz, const uint8_t* sign,
                             const DpufGemvJob* job, int32_t* flags, const int32_t* serial) {
    MvKernel kf;
    int threads, np, nwg;
    size_t lds;
    if (!flags || !serial || !fed_plan(I, job, kf, threads, np, nwg, lds)) return -1;
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
    A.wb[0] = 0;
    A.wb[1] = nwg;
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
    hipLaunchKernelGGL(kf, dim3(np + nwg), dim3(threads), lds, ST(s), A);
    LAUNCHED("k_mv");
    return 0;
}

void dpuf_hip_gemv_zero(void* s, int32_t M, const DpufGemvJob* job, int32_t r0, int32_t r1) {
    if (M == 1) {
        dpuf_hip_gemv(s, 1, 1, job, NULL, 0.0f);
        if (r1 > r0) dpuf_hip_zero_rows(s, 1, job->out, job->ldo, r0, r1);
        return;
    }
    dpuf_hip_gm_launch(s, M, 1, job, job->out, job->ldo, r0, r1);
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
            if (dpuf_hip_mvt_launch(s, M, n, sub) != 0) dpuf_hip_gm_launch(s, M, n, sub, NULL, 0, 0, 0);
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


int32_t dpuf_hip_gemv_red(void* s, const DpufGemvJob* job, const int32_t* skip_flag, float fill, void* red,
                          int32_t red_cap) {
    const int mode = job->w.mode;
    if ((mode != 12 && mode != 13 && mode != 14) || !red || red_cap <= 0) {
        note(hipErrorInvalidValue, "dpuf_hip_gemv_red: bad arguments");
        return -1;
    }
    MvArgs A;
    memset(&A, 0, sizeof A);
    A.n_jobs = 1;
    A.K = job->w.cols;
    A.j[0].g = job->w.g;
    A.j[0].out = job->out;
    A.j[0].g0 = job->g0;
    A.j[0].g1 = job->g1;
    A.j[0].rows = job->w.rows;
    A.j[0].x = job->p;
    A.skip_flag = skip_flag;
    A.fill = fill;
    A.red = (lm4*)red;
    const int ng = job->g1 - job->g0 > 0 ? job->g1 - job->g0 : 0;
    return mv_launch(s, A, &ng, mode, red_cap);
}

int dpuf_hip_mv_max_wg(void) { return g_mv_max_wg; }

}  // extern "C"
