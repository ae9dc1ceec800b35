/*
 * oracle.c -- CPU restatement of the reference DPUF token loop: the Mode 12
 * (Hadamard-4bit packed) path and the asymmetric blk64 Modes 13 / 14.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
 * this file: it is the checker that tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py compare the HIP engine against.
 *
 * Every function restates the arithmetic of the reference in portable C, with
 * the same fp32 operation order, so that outputs are bit-comparable:
 *   - 8-wide SIMD accumulators become explicit 8-element arrays;
 *   - _mm256_fmadd_ps becomes fmaf (build with -ffp-contract=off so that no
 *     other multiply-add is fused);
 *   - horizontal sums use the exact trees of the reference's hsum/hadd code.
 * Each function cites the reference file:line it follows.
 *
 * Known, documented deviations (none reachable at the shapes used here):
 *   - SwiGLU always takes the 8-wide path (reference dpuf_engine.c:976-989); the
 *     scalar tail (dpuf_engine.c:990-996) only runs when a thread's slice is not
 *     a multiple of 8, which never happens for n_threads in {1,2,4,8} and
 *     intermediate sizes that are multiples of 64.
 *   - RMSNorm / dot scalar tails (n % 8 != 0) are not restated; all dims are
 *     multiples of 8.
 *   - The scalar expression of Modes 13 / 14, xm_s = (a * b + c * d) * 0.125f
 *     (dpuf_avx2.c:2877, 3031), is evaluated unfused, as the reference's
 *     Linux build (Makefile: gcc -std=c11, whose default is
 *     -ffp-contract=off) compiles it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#include "oracle.h"

/* ------------------------------------------------------------------------- */
/* Scalars                                                                    */
/* ------------------------------------------------------------------------- */

/* IEEE binary16 -> binary32, exact (same values as F16C vcvtph2ps used at
 * reference dpuf_avx2.c:705-707, 2509, 2634). */
float orc_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* Sum of an 8-lane accumulator in the order of eng_hsum256_ps
 * (reference dpuf_engine.c:37-46): ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)). */
static inline float hsum8(const float a[8]) {
    float s0 = a[0] + a[4], s1 = a[1] + a[5], s2 = a[2] + a[6], s3 = a[3] + a[7];
    return (s0 + s1) + (s2 + s3);
}

/* Sum of one 8-lane accumulator as produced by hsum4_256_ps's two hadd levels
 * plus the final low+high add (reference dpuf_engine.c:318-323):
 * ((a0+a1)+(a2+a3)) + ((a4+a5)+(a6+a7)). */
static inline float hsum8_hadd(const float a[8]) {
    float lo = (a[0] + a[1]) + (a[2] + a[3]);
    float hi = (a[4] + a[5]) + (a[6] + a[7]);
    return lo + hi;
}

/* 8-wide exp polynomial of the reference (dpuf_engine.c:297-316), lane-wise. */
float orc_exp_poly(float x) {
    const float ln2_hi = 0.693359375f;
    const float ln2_lo = -2.12194440e-4f;
    const float inv_ln2 = 1.44269504088896341f;
    x = fmaxf(-45.0f, fminf(x, 45.0f));
    float fx = rintf(x * inv_ln2);
    float r = fmaf(-fx, ln2_hi, x);
    r = fmaf(-fx, ln2_lo, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    float er = fmaf(p, r2, r) + 1.0f;
    int32_t n = (int32_t)fx;
    uint32_t bits = (uint32_t)(n + 127) << 23;
    float sc;
    memcpy(&sc, &bits, 4);
    return er * sc;
}

/* ------------------------------------------------------------------------- */
/* A1: FWHT-64 and sign mask (reference dpuf_avx2.c:709-788)                  */
/* ------------------------------------------------------------------------- */

/* In-place radix-2 butterflies with strides 1,2,4,8,16,32 then x 0.125
 * (reference fwht64_block_f32, dpuf_avx2.c:724-772). */
void orc_fwht64(float* y) {
    for (int h = 1; h < 64; h <<= 1) {
        for (int i = 0; i < 64; i += (h << 1)) {
            for (int j = i; j < i + h; j++) {
                float a = y[j], b = y[j + h];
                y[j] = a + b;
                y[j + h] = a - b;
            }
        }
    }
    for (int i = 0; i < 64; i++) y[i] = y[i] * 0.125f;
}

/* Reference dpuf_fwht64_sign_f32 (dpuf_avx2.c:774-788). */
void orc_fwht64_sign(int32_t cols, const float* x, const uint8_t* sb, float* out) {
    for (int32_t c = 0; c < cols; c++) {
        float v = x[c];
        if (sb && ((sb[c >> 3] >> (c & 7)) & 1u)) v = -v;
        out[c] = v;
    }
    for (int32_t c = 0; c < cols; c += 64) orc_fwht64(out + c);
}

/* ------------------------------------------------------------------------- */
/* A2: activation prep (reference dpuf_prep_had4_packed_slab, 2364-2449)     */
/* ------------------------------------------------------------------------- */

/* Quantises one 32-block of FWHT'd values: returns scale, writes q and sum8. */
static float quant_block32(const float* f, int8_t* q, int32_t* sum8) {
    float amax = 0.0f;
    for (int k = 0; k < 32; k++) {
        float a = fabsf(f[k]);
        amax = (a > amax) ? a : amax;
    }
    if (amax <= 1e-4f) {
        memset(q, 0, 32);
        *sum8 = 0;
        return 0.0f;
    }
    float d = amax / 127.0f;
    float inv = (amax > 1e-12f) ? (127.0f / amax) : 0.0f;
    int32_t s = 0;
    for (int k = 0; k < 32; k++) {
        float v = f[k] * inv;
        /* cvtps_epi32 (RNE, out-of-range/NaN -> INT_MIN), packs to i16/i8
         * with saturation, then max with -127 (dpuf_avx2.c:2420-2426). */
        int32_t qi;
        if (!(v > -2147483648.0f && v < 2147483648.0f)) qi = INT32_MIN;
        else qi = (int32_t)rintf(v);
        if (qi > 127) qi = 127;
        if (qi < -128) qi = -128;
        if (qi < -127) qi = -127;
        q[k] = (int8_t)qi;
        s += qi;
    }
    *sum8 = s * 8;
    return d;
}

/* Row layout (pack_slab = 0): q[cols], scale[n_blk], sum8[n_blk]. */
void orc_prep_row(int32_t cols, const float* x, const uint8_t* sb,
                  int8_t* q, float* scale, int32_t* sum8) {
    float* f = (float*)malloc((size_t)cols * sizeof(float));
    orc_fwht64_sign(cols, x, sb, f);
    for (int32_t b = 0; b < (cols >> 5); b++) {
        scale[b] = quant_block32(f + 32 * b, q + 32 * b, sum8 + b);
    }
    free(f);
}

/* Slab layout (pack_slab = 1) for mc <= 6 rows: words [n_blk][8][6],
 * scales/sums [n_blk][6] (dpuf_avx2.c:2390-2447).  Unused token lanes of a
 * partial slab are left untouched, as in the reference. */
void orc_prep_slab(int32_t mc, int32_t cols, const float* x, const uint8_t* sb,
                   int8_t* xq_slab, float* scale, int32_t* sum8) {
    int32_t n_blk = cols >> 5;
    int8_t* q = (int8_t*)malloc((size_t)cols);
    float* s = (float*)malloc((size_t)n_blk * sizeof(float));
    int32_t* m = (int32_t*)malloc((size_t)n_blk * sizeof(int32_t));
    for (int32_t j = 0; j < mc; j++) {
        orc_prep_row(cols, x + (size_t)j * cols, sb, q, s, m);
        for (int32_t b = 0; b < n_blk; b++) {
            int32_t* words = (int32_t*)(xq_slab + (size_t)b * 192u);
            for (int g = 0; g < 8; g++) {
                int32_t w;
                memcpy(&w, q + 32 * b + 4 * g, 4);
                words[g * 6 + j] = w;
            }
            scale[(size_t)b * 6 + j] = s[b];
            sum8[(size_t)b * 6 + j] = m[b];
        }
    }
    free(q); free(s); free(m);
}

/* ------------------------------------------------------------------------- */
/* A3/A4: Mode 12 GEMV / GEMM (reference dpuf_avx2.c:2585-2676)               */
/* ------------------------------------------------------------------------- */

/* Integer dot of row ri of one 144-byte (8 rows x 32 cols) group-block with
 * int8 activations of that block: sum_k u_k * q_k, exact. */
static inline int32_t group_block_dot(const uint8_t* qp, int ri, const int8_t* xq) {
    int32_t d = 0;
    for (int c = 0; c < 4; c++) {
        const uint8_t* cp = qp + c * 32 + ri * 4;
        for (int k = 0; k < 4; k++) {
            d += (int32_t)(cp[k] & 0x0Fu) * (int32_t)xq[8 * c + k];
            d += (int32_t)(cp[k] >> 4) * (int32_t)xq[8 * c + 4 + k];
        }
    }
    return d;
}

/* Computes rows of tiles [t0, t1) for M tokens whose activations were prepped
 * in row layout (xq [M][cols], xs/xsum [M][n_blk]).  out is [M][rows].
 * skip_zero_blocks reproduces the M == 1 branch (dpuf_avx2.c:2621-2622);
 * the slab branch (M > 1) accumulates every block.  For each (row, token):
 *   acc = fma(float(D - sum8), fp16(ws) * xs, acc), blocks ascending. */
void orc_gemm_tiles(int32_t M, int32_t rows, int32_t cols, int32_t t0, int32_t t1,
                    const int8_t* xq, const float* xs, const int32_t* xsum,
                    const uint8_t* base, const uint64_t* offs, float* out,
                    int skip_zero_blocks) {
    const int32_t n_blk = cols >> 5;
    int32_t t;
#pragma omp parallel for schedule(static) if (t1 - t0 >= 8)
    for (t = t0; t < t1; t++) {
        const uint8_t* tp = base + offs[t];
        const DpufQrTileHdr* th = (const DpufQrTileHdr*)tp;
        int32_t n_r = th->n_rows;
        int32_t n_8g = (n_r + 7) >> 3;
        for (int32_t rg = 0; rg < n_8g; rg++) {
            int32_t n_8 = (rg * 8 + 8 <= n_r) ? 8 : (n_r - rg * 8);
            const uint8_t* grp = tp + sizeof(DpufQrTileHdr) + (size_t)rg * (size_t)n_blk * 144u;
            const uint16_t* sc = (const uint16_t*)grp;
            const uint8_t* qg = grp + (size_t)n_blk * 16u;
            for (int32_t m = 0; m < M; m++) {
                const int8_t* xm = xq + (size_t)m * cols;
                const float* sm = xs + (size_t)m * n_blk;
                const int32_t* um = xsum + (size_t)m * n_blk;
                for (int ri = 0; ri < n_8; ri++) {
                    float acc = 0.0f;
                    for (int32_t b = 0; b < n_blk; b++) {
                        float bs = sm[b];
                        if (skip_zero_blocks && bs <= 0.0f) continue;
                        int32_t d = group_block_dot(qg + (size_t)b * 128u, ri, xm + 32 * b) - um[b];
                        float ws = orc_h2f(sc[(size_t)b * 8u + ri]);
                        acc = fmaf((float)d, ws * bs, acc);
                    }
                    out[(size_t)m * rows + (size_t)t * 16 + rg * 8 + ri] = acc;
                }
            }
        }
    }
}

/* Standalone fp32 entry (reference dpuf_matmul_qr_hadamard4_packed_f32,
 * dpuf_avx2.c:2678-2736). */
void orc_matmul_f32(int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                    const float* x, const uint8_t* base, const uint64_t* offs,
                    const uint8_t* sb, float* out) {
    int32_t n_blk = cols >> 5;
    int8_t* q = (int8_t*)malloc((size_t)M * cols);
    float* s = (float*)malloc((size_t)M * n_blk * sizeof(float));
    int32_t* m = (int32_t*)malloc((size_t)M * n_blk * sizeof(int32_t));
    for (int32_t i = 0; i < M; i++) {
        orc_prep_row(cols, x + (size_t)i * cols, sb, q + (size_t)i * cols,
                     s + (size_t)i * n_blk, m + (size_t)i * n_blk);
    }
    orc_gemm_tiles(M, rows, cols, 0, n_tiles, q, s, m, base, offs, out, M == 1);
    free(q); free(s); free(m);
}

/* ------------------------------------------------------------------------- */
/* A6: embedding (reference dpuf_avx2.c:2738-2783)                            */
/* ------------------------------------------------------------------------- */

void orc_embed(int32_t n_tokens, int32_t cols, const int32_t* ids,
               const uint8_t* base, const uint64_t* offs, const uint8_t* sb, float* out) {
    const int32_t n_blk = cols >> 5;
    for (int32_t i = 0; i < n_tokens; i++) {
        int32_t r = ids[i];
        int32_t t = r / 16, lr = r % 16, rg = lr >> 3, ri = lr & 7;
        const uint8_t* grp = base + offs[t] + sizeof(DpufQrTileHdr) + (size_t)rg * (size_t)n_blk * 144u;
        const uint16_t* sc = (const uint16_t*)grp;
        const uint8_t* qg = grp + (size_t)n_blk * 16u;
        float* dst = out + (size_t)i * cols;
        for (int32_t b = 0; b < n_blk; b++) {
            float ws = orc_h2f(sc[(size_t)b * 8u + ri]);
            for (int c = 0; c < 4; c++) {
                const uint8_t* cp = qg + (size_t)b * 128u + c * 32 + ri * 4;
                for (int k = 0; k < 4; k++) {
                    dst[32 * b + 8 * c + k] = (float)((int32_t)(cp[k] & 0x0Fu) - 8) * ws;
                    dst[32 * b + 8 * c + 4 + k] = (float)((int32_t)(cp[k] >> 4) - 8) * ws;
                }
            }
        }
        for (int32_t c = 0; c < cols; c += 64) orc_fwht64(dst + c);
        if (sb) {
            for (int32_t c = 0; c < cols; c++) {
                if ((sb[c >> 3] >> (c & 7)) & 1u) dst[c] = -dst[c];
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Modes 13 / 14: asymmetric blk64 4-bit and 6-bit (reference                 */
/* dpuf_avx2.c:2785-3221)                                                     */
/* ------------------------------------------------------------------------- */

/* A tile's 8-row group g (rows 8g .. 8g+7) holds, for n_64 = cols/64 blocks of
 * 64 columns (dpuf_avx2.c:2786-2791, dpuf_format.py:1699-1725):
 *   dm  [n_64][16] fp16: d of rows 0..7, then m of rows 0..7;
 *   q4  [n_blk][128] bytes, the mode 12 nibble interleave: byte c*32 + ri*4 + k
 *       of 32-block b holds row ri, column 32b+8c+k (low nibble) and 32b+8c+4+k
 *       (high nibble);
 *   q2  (mode 14 only) [n_blk][64] bytes: bits 2(ri>>1) .. +1 of byte
 *       c*16 + h*8 + (ri&1)*4 + k are bits 4..5 of row ri, column 32b+8c+4h+k.
 * Group bytes per 64 columns: 288 (mode 13), 416 (mode 14). */
static size_t asym_grp_bytes(int is_had6, int32_t n_64) { return (size_t)n_64 * (is_had6 ? 416u : 288u); }

/* Quantised value u of row ri, column j (0..31) of one 32-block. */
static inline int32_t asym_u(const uint8_t* qp, const uint8_t* h2p, int ri, int j) {
    const int c = j >> 3, h = (j >> 2) & 1, k = j & 3;
    const uint8_t by = qp[c * 32 + ri * 4 + k];
    int32_t u = h ? (by >> 4) : (by & 0x0F);
    if (h2p) u |= ((h2p[c * 16 + h * 8 + (ri & 1) * 4 + k] >> ((ri >> 1) * 2)) & 3) << 4;
    return u;
}

/* Exact integer dot of row ri of one 32-block with int8 activations: the
 * reference's maddubs / madd sums (dpuf_avx2.c:2802-2846) never saturate or
 * wrap, since |u q| <= 63 * 127 and at most 8 products share an int16 lane. */
static inline int32_t asym_block_dot(const uint8_t* qp, const uint8_t* h2p, int ri, const int8_t* xq) {
    int32_t d = 0;
    for (int j = 0; j < 32; j++) d += asym_u(qp, h2p, ri, j) * (int32_t)xq[j];
    return d;
}

/* Rows of tiles [t0, t1) for M tokens prepped in row layout (as
 * orc_gemm_tiles).  For each (row, token), over 64-blocks g ascending
 * (dpuf_avx2.c:3029-3037 for M == 1, 2871-2882 for the slabs, identical):
 *   fdot = fma(float(D0), xs0, float(D1) * xs1)
 *   xm_s = ((float)sum8_0 * xs0 + (float)sum8_1 * xs1) * 0.125f   (no fusion)
 *   acc  = fma(fdot, d, acc);  acc = fma(m, xm_s, acc)
 * with D0, D1 the dots of 32-blocks 2g, 2g+1.  No block is skipped. */
void orc_gemm_tiles_asym(int32_t is_had6, int32_t M, int32_t rows, int32_t cols, int32_t t0, int32_t t1,
                         const int8_t* xq, const float* xs, const int32_t* xsum,
                         const uint8_t* base, const uint64_t* offs, float* out) {
    const int32_t n_blk = cols >> 5, n_64 = cols >> 6;
    const size_t gbytes = asym_grp_bytes(is_had6, n_64);
    int32_t t;
#pragma omp parallel for schedule(static) if (t1 - t0 >= 8)
    for (t = t0; t < t1; t++) {
        const uint8_t* tp = base + offs[t];
        const DpufQrTileHdr* th = (const DpufQrTileHdr*)tp;
        int32_t n_r = th->n_rows;
        int32_t n_8g = (n_r + 7) >> 3;
        for (int32_t rg = 0; rg < n_8g; rg++) {
            int32_t n_8 = (rg * 8 + 8 <= n_r) ? 8 : (n_r - rg * 8);
            const uint8_t* grp = tp + sizeof(DpufQrTileHdr) + (size_t)rg * gbytes;
            const uint16_t* dm = (const uint16_t*)grp;
            const uint8_t* q4 = grp + (size_t)n_64 * 32u;
            const uint8_t* q2 = is_had6 ? q4 + (size_t)n_64 * 256u : NULL;
            for (int32_t m = 0; m < M; m++) {
                const int8_t* xm = xq + (size_t)m * cols;
                const float* sm = xs + (size_t)m * n_blk;
                const int32_t* um = xsum + (size_t)m * n_blk;
                for (int ri = 0; ri < n_8; ri++) {
                    float acc = 0.0f;
                    for (int32_t g = 0; g < n_64; g++) {
                        const int32_t b0 = 2 * g, b1 = b0 + 1;
                        const int32_t d0 = asym_block_dot(q4 + (size_t)b0 * 128u, q2 ? q2 + (size_t)b0 * 64u : NULL,
                                                          ri, xm + 32 * b0);
                        const int32_t d1 = asym_block_dot(q4 + (size_t)b1 * 128u, q2 ? q2 + (size_t)b1 * 64u : NULL,
                                                          ri, xm + 32 * b1);
                        const float xs0 = sm[b0], xs1 = sm[b1];
                        const float fdot = fmaf((float)d0, xs0, (float)d1 * xs1);
                        const float xm_s = ((float)um[b0] * xs0 + (float)um[b1] * xs1) * 0.125f;
                        const float wd = orc_h2f(dm[(size_t)g * 16u + ri]);
                        const float wm = orc_h2f(dm[(size_t)g * 16u + 8u + ri]);
                        acc = fmaf(fdot, wd, acc);
                        acc = fmaf(wm, xm_s, acc);
                    }
                    out[(size_t)m * rows + (size_t)t * 16 + rg * 8 + ri] = acc;
                }
            }
        }
    }
}

/* Standalone fp32 entries (reference had_asym_matmul_f32_impl,
 * dpuf_avx2.c:3084-3136): the mode 12 prep, then the tiles above. */
void orc_matmul_asym_f32(int32_t is_had6, int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                         const float* x, const uint8_t* base, const uint64_t* offs,
                         const uint8_t* sb, float* out) {
    int32_t n_blk = cols >> 5;
    int8_t* q = (int8_t*)malloc((size_t)M * cols);
    float* s = (float*)malloc((size_t)M * n_blk * sizeof(float));
    int32_t* m = (int32_t*)malloc((size_t)M * n_blk * sizeof(int32_t));
    for (int32_t i = 0; i < M; i++)
        orc_prep_row(cols, x + (size_t)i * cols, sb, q + (size_t)i * cols, s + (size_t)i * n_blk, m + (size_t)i * n_blk);
    orc_gemm_tiles_asym(is_had6, M, rows, cols, 0, n_tiles, q, s, m, base, offs, out);
    free(q); free(s); free(m);
}

/* Embedding rows (reference embed_qr_had_asym_impl, dpuf_avx2.c:3154-3207):
 * value (float)u * d + m (a rounded product, then a rounded sum), FWHT-64
 * per 64 columns, then the signs. */
void orc_embed_asym(int32_t is_had6, int32_t n_tokens, int32_t cols, const int32_t* ids,
                    const uint8_t* base, const uint64_t* offs, const uint8_t* sb, float* out) {
    const int32_t n_64 = cols >> 6;
    const size_t gbytes = asym_grp_bytes(is_had6, n_64);
    for (int32_t i = 0; i < n_tokens; i++) {
        int32_t r = ids[i];
        int32_t t = r / 16, lr = r % 16, rg = lr >> 3, ri = lr & 7;
        const uint8_t* grp = base + offs[t] + sizeof(DpufQrTileHdr) + (size_t)rg * gbytes;
        const uint16_t* dm = (const uint16_t*)grp;
        const uint8_t* q4 = grp + (size_t)n_64 * 32u;
        const uint8_t* q2 = is_had6 ? q4 + (size_t)n_64 * 256u : NULL;
        float* dst = out + (size_t)i * cols;
        for (int32_t g = 0; g < n_64; g++) {
            const float wd = orc_h2f(dm[(size_t)g * 16u + ri]);
            const float wm = orc_h2f(dm[(size_t)g * 16u + 8u + ri]);
            for (int sub = 0; sub < 2; sub++) {
                const int32_t b = 2 * g + sub;
                const uint8_t* qp = q4 + (size_t)b * 128u;
                const uint8_t* hp = q2 ? q2 + (size_t)b * 64u : NULL;
                for (int j = 0; j < 32; j++) {
                    const float pr = (float)asym_u(qp, hp, ri, j) * wd;
                    dst[32 * b + j] = pr + wm;
                }
            }
        }
        for (int32_t c = 0; c < cols; c += 64) orc_fwht64(dst + c);
        if (sb) {
            for (int32_t c = 0; c < cols; c++) {
                if ((sb[c >> 3] >> (c & 7)) & 1u) dst[c] = -dst[c];
            }
        }
    }
}

/* Embedding of any supported mode (reference dpuf_embed_qr_any_f32,
 * dpuf_avx2.c:2044-2067). */
void orc_embed_desc(const DpufWeightDesc* w, int32_t n_tokens, const int32_t* ids, float* out) {
    if (w->mode == DPUF_MODE_QR_HAD4_PACKED)
        orc_embed(n_tokens, w->cols, ids, w->tensor_base, w->tile_offsets, w->sign_bits, out);
    else if (w->mode == DPUF_MODE_QR_HAD4_ASYM || w->mode == DPUF_MODE_QR_HAD6)
        orc_embed_asym(w->mode == DPUF_MODE_QR_HAD6, n_tokens, w->cols, ids, w->tensor_base, w->tile_offsets,
                       w->sign_bits, out);
}

/* ------------------------------------------------------------------------- */
/* A8: RMSNorm (reference dpuf_engine.c:225-272)                              */
/* ------------------------------------------------------------------------- */

/* Summation order of the RMSNorm sum of squares: 0 the reference's (eight
 * fma lanes + hsum8), 1 a pairwise tree of the squares.  Test
 * infrastructure only: the order-sensitivity test measures how far a
 * reordered but equally valid fp32 sum moves logits and greedy ids. */
static int g_norm_tree = 0;
void orc_set_norm_order(int32_t tree) { g_norm_tree = tree; }

static float tree_sum(const float* v, int32_t n) {
    if (n == 1) return v[0];
    const int32_t h = n / 2;
    return tree_sum(v, h) + tree_sum(v + h, n - h);
}

/* x += res (when res != NULL, stored back), out = (x * inv) * w with
 * inv = 1 / sqrtf(ss / n + eps), ss from eight fma lanes + hsum8. */
void orc_add_rmsnorm(int32_t n, float* x, const float* res, const float* w, float eps, float* out) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int32_t i = 0; i + 7 < n; i += 8) {
        for (int j = 0; j < 8; j++) {
            float s = res ? (x[i + j] + res[i + j]) : x[i + j];
            if (res) x[i + j] = s;
            acc[j] = fmaf(s, s, acc[j]);
        }
    }
    float ss = hsum8(acc);
    if (g_norm_tree && n > 0) {
        float* sq = (float*)malloc((size_t)n * sizeof(float));
        for (int32_t i = 0; i < n; i++) sq[i] = x[i] * x[i];
        ss = tree_sum(sq, n);
        free(sq);
    }
    float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (int32_t i = 0; i < n; i++) out[i] = (x[i] * inv) * w[i];
}

/* ------------------------------------------------------------------------- */
/* A9: RoPE (reference dpuf_engine.c:183-223, 274-295)                        */
/* ------------------------------------------------------------------------- */

void orc_rope_tables(const DpufModelConfig* cfg, float* cos_tab, float* sin_tab) {
    int32_t hd = cfg->head_dim, half = hd >> 1;
    float* inv_freq = (float*)malloc((size_t)half * sizeof(float));
    for (int32_t j = 0; j < half; j++) {
        float freq = 1.0f / powf(cfg->rope_theta, (float)(2 * j) / (float)hd);
        if (cfg->use_llama3_rope) {
            float factor = cfg->rope_factor, low_f = cfg->rope_low_freq, high_f = cfg->rope_high_freq;
            float orig_max = (float)cfg->rope_orig_max_pos;
            float wavelen = (2.0f * 3.14159265358979323846f) / freq;
            float low_wavelen = orig_max / low_f, high_wavelen = orig_max / high_f;
            if (wavelen > low_wavelen) {
                freq /= factor;
            } else if (wavelen >= high_wavelen) {
                float smooth = (orig_max / wavelen - low_f) / (high_f - low_f);
                freq = (1.0f - smooth) * (freq / factor) + smooth * freq;
            }
        }
        inv_freq[j] = freq;
    }
    for (int32_t p = 0; p < cfg->max_seq_len; p++) {
        for (int32_t j = 0; j < half; j++) {
            float ang = (float)p * inv_freq[j];
            cos_tab[(size_t)p * half + j] = cosf(ang);
            sin_tab[(size_t)p * half + j] = sinf(ang);
        }
    }
    free(inv_freq);
}

/* NeoX half rotation with fmsub/fmadd (dpuf_engine.c:274-284). */
void orc_rope_apply(int32_t hd, float* v, const float* c, const float* s) {
    int32_t half = hd >> 1;
    for (int32_t j = 0; j < half; j++) {
        float x1 = v[j], x2 = v[j + half];
        float o1 = fmaf(x1, c[j], -(x2 * s[j]));
        float o2 = fmaf(x2, c[j], x1 * s[j]);
        v[j] = o1;
        v[j + half] = o2;
    }
}

/* ------------------------------------------------------------------------- */
/* A10: attention over the fp32 KV cache (reference dpuf_engine.c:325-577)    */
/* ------------------------------------------------------------------------- */

/* Softmax with the vector/tail split of dpuf_engine.c:409-431. */
static void softmax_ref(int32_t n, float* sc, float mx) {
    float vs[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int32_t k = 0;
    for (; k + 7 < n; k += 8) {
        for (int j = 0; j < 8; j++) {
            float e = orc_exp_poly(sc[k + j] - mx);
            sc[k + j] = e;
            vs[j] = vs[j] + e;
        }
    }
    float sp = hsum8(vs);
    for (; k < n; k++) {
        float e = expf(sc[k] - mx);
        sc[k] = e;
        sp += e;
    }
    float inv = 1.0f / (sp + 1e-12f);
    for (k = 0; k < n; k++) sc[k] = sc[k] * inv;
}

/* Scores of one query against keys [0, kv_len) with the reference's grouping:
 * keys in blocks of four use the hadd tree, the remainder uses hsum8. */
static float scores_ref(int32_t hd, int32_t kv_len, float scale, const float* kc,
                        const float* q, float* sc, int single_head_tail) {
    float mx = -1e30f;
    int32_t t = 0;
    for (; t + 3 < kv_len; t += 4) {
        for (int u = 0; u < 4; u++) {
            const float* kp = kc + (size_t)(t + u) * hd;
            float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int32_t i = 0; i < hd; i += 8)
                for (int j = 0; j < 8; j++) a[j] = fmaf(q[i + j], kp[i + j], a[j]);
            float s = hsum8_hadd(a) * scale;
            sc[t + u] = s;
            mx = (s > mx) ? s : mx;
        }
    }
    for (; t < kv_len; t++) {
        const float* kp = kc + (size_t)t * hd;
        float s;
        if (!single_head_tail) {
            float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int32_t i = 0; i < hd; i += 8)
                for (int j = 0; j < 8; j++) a[j] = fmaf(q[i + j], kp[i + j], a[j]);
            s = hsum8(a) * scale;
        } else {
            /* dot_f32_avx2 (dpuf_engine.c:325-339): two accumulators over
             * 16-wide steps, then an 8-wide step, summed lane-wise first. */
            float a0[8] = {0, 0, 0, 0, 0, 0, 0, 0}, a1[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            int32_t i = 0;
            for (; i + 15 < hd; i += 16)
                for (int j = 0; j < 8; j++) {
                    a0[j] = fmaf(q[i + j], kp[i + j], a0[j]);
                    a1[j] = fmaf(q[i + 8 + j], kp[i + 8 + j], a1[j]);
                }
            for (; i + 7 < hd; i += 8)
                for (int j = 0; j < 8; j++) a0[j] = fmaf(q[i + j], kp[i + j], a0[j]);
            float c[8];
            for (int j = 0; j < 8; j++) c[j] = a0[j] + a1[j];
            s = hsum8(c) * scale;
        }
        sc[t] = s;
        if (s > mx) mx = s;
    }
    return mx;
}

/* gqa_attn_head_pair_f32 (dpuf_engine.c:341-577) for hd % 8 == 0.
 * q1 == NULL selects the single-head path. */
void orc_attn_heads(int32_t hd, int32_t kv_len, float scale, const float* kc, const float* vc,
                    const float* q0, const float* q1, float* sc0, float* sc1,
                    float* out0, float* out1) {
    if (q1) {
        float m0 = scores_ref(hd, kv_len, scale, kc, q0, sc0, 0);
        float m1 = scores_ref(hd, kv_len, scale, kc, q1, sc1, 0);
        softmax_ref(kv_len, sc0, m0);
        softmax_ref(kv_len, sc1, m1);
        for (int32_t d = 0; d < hd; d++) {
            float a = 0.0f, b = 0.0f;
            for (int32_t k = 0; k < kv_len; k++) {
                float v = vc[(size_t)k * hd + d];
                a = fmaf(sc0[k], v, a);
                b = fmaf(sc1[k], v, b);
            }
            out0[d] = a;
            out1[d] = b;
        }
        return;
    }
    float m0 = scores_ref(hd, kv_len, scale, kc, q0, sc0, 1);
    softmax_ref(kv_len, sc0, m0);
    if ((hd & 63) == 0) {
        /* Pairs of keys: a = fma(p_k, v_k, fma(p_k+1, v_k+1, a)) (dpuf_engine.c:535-558). */
        for (int32_t d = 0; d < hd; d++) {
            float a = 0.0f;
            int32_t k = 0;
            for (; k + 1 < kv_len; k += 2)
                a = fmaf(sc0[k], vc[(size_t)k * hd + d], fmaf(sc0[k + 1], vc[(size_t)(k + 1) * hd + d], a));
            if (k < kv_len) a = fmaf(sc0[k], vc[(size_t)k * hd + d], a);
            out0[d] = a;
        }
    } else {
        for (int32_t d = 0; d < hd; d++) {
            float a = 0.0f;
            for (int32_t k = 0; k < kv_len; k++) a = fmaf(sc0[k], vc[(size_t)k * hd + d], a);
            out0[d] = a;
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Q8 KV cache (kv_type 1): per-32 int8 K/V and its attention                 */
/* (reference dpuf_engine.c:579-781)                                          */
/* ------------------------------------------------------------------------- */

/* quantize_vec_q8_blk32 (dpuf_engine.c:754-781): per 32-block amax,
 * scale = amax / 127, q = RNE(v * (127 / amax)) saturated and clamped to
 * >= -127 (a value the conversion cannot represent becomes -127, as
 * cvtps_epi32's 0x80000000 does after the saturating packs); amax <= 1e-12
 * gives q = 0 with scale amax / 127. */
void orc_quant_q8(int32_t n, const float* src, int8_t* dst, float* scales) {
    for (int32_t b = 0; b < (n >> 5); b++) {
        const float* v = src + 32 * b;
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = fabsf(v[j]);
            amax = a > amax ? a : amax;
        }
        scales[b] = amax / 127.0f;
        const float inv = (amax > 1e-12f) ? (127.0f / amax) : 0.0f;
        for (int j = 0; j < 32; j++) {
            const float x = v[j] * inv;
            int32_t q;
            if (!(x > -2147483648.0f && x < 2147483648.0f)) q = -127;
            else q = (int32_t)rintf(x);
            q = q > 127 ? 127 : q;
            q = q < -127 ? -127 : q;
            dst[32 * b + j] = (int8_t)q;
        }
    }
}

/* dot_f32_q8_blk32_avx2 (dpuf_engine.c:579-593): per block two 8-lane
 * accumulators (columns 0-7 then 16-23, and 8-15 then 24-31), their lane sum
 * scaled into a running 8-lane total, then eng_hsum256. */
static float dot_q8(int32_t hd, const float* q, const int8_t* k, const float* ks) {
    float tot[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int32_t b = 0; b < (hd >> 5); b++) {
        const int32_t c0 = 32 * b;
        for (int L = 0; L < 8; L++) {
            float a0 = fmaf(q[c0 + L], (float)k[c0 + L], 0.0f);
            float a1 = fmaf(q[c0 + 8 + L], (float)k[c0 + 8 + L], 0.0f);
            a0 = fmaf(q[c0 + 16 + L], (float)k[c0 + 16 + L], a0);
            a1 = fmaf(q[c0 + 24 + L], (float)k[c0 + 24 + L], a1);
            tot[L] = fmaf(a0 + a1, ks[b], tot[L]);
        }
    }
    return hsum8(tot);
}

/* The pair path's score of one query against one key (dpuf_engine.c:611-648):
 * per block, lanes accumulate fma(q_lo, k_lo, fma(q_hi, k_hi, t)) over the two
 * 16-column halves, then fma(t, ks, s); the hadd tree of hsum4_256_ps. */
static float pair_score_q8(int32_t hd, const float* q, const int8_t* k, const float* ks) {
    float sa[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int32_t b = 0; b < (hd >> 5); b++) {
        const int32_t c0 = 32 * b;
        for (int L = 0; L < 8; L++) {
            float t = 0.0f;
            for (int j = 0; j < 32; j += 16)
                t = fmaf(q[c0 + j + L], (float)k[c0 + j + L], fmaf(q[c0 + j + 8 + L], (float)k[c0 + j + 8 + L], t));
            sa[L] = fmaf(t, ks[b], sa[L]);
        }
    }
    return hsum8_hadd(sa);
}

/* gqa_attn_head_pair_q8 (dpuf_engine.c:595-752) over a head's int8 K/V
 * [kv_len][hd] and per-32 scales [kv_len][hd/32].  q1 == NULL selects the
 * single-head path. */
void orc_attn_heads_q8(int32_t hd, int32_t kv_len, float scale, const int8_t* kq, const float* ks,
                       const int8_t* vq, const float* vs, const float* q0, const float* q1,
                       float* sc0, float* sc1, float* out0, float* out1) {
    const int32_t nb = hd >> 5;
    float m0 = -1e30f, m1 = -1e30f;
    if (q1) {
        int32_t t = 0;
        for (; t + 1 < kv_len; t += 2) {
            for (int u = 0; u < 2; u++) {
                const int8_t* kp = kq + (size_t)(t + u) * hd;
                const float* kps = ks + (size_t)(t + u) * nb;
                sc0[t + u] = pair_score_q8(hd, q0, kp, kps) * scale;
                sc1[t + u] = pair_score_q8(hd, q1, kp, kps) * scale;
            }
            const float a = sc0[t] > sc0[t + 1] ? sc0[t] : sc0[t + 1];
            const float c = sc1[t] > sc1[t + 1] ? sc1[t] : sc1[t + 1];
            m0 = a > m0 ? a : m0;
            m1 = c > m1 ? c : m1;
        }
        for (; t < kv_len; t++) {
            const int8_t* kp = kq + (size_t)t * hd;
            const float* kps = ks + (size_t)t * nb;
            const float s0 = dot_q8(hd, q0, kp, kps) * scale, s1 = dot_q8(hd, q1, kp, kps) * scale;
            sc0[t] = s0;
            if (s0 > m0) m0 = s0;
            sc1[t] = s1;
            if (s1 > m1) m1 = s1;
        }
        softmax_ref(kv_len, sc0, m0);
        softmax_ref(kv_len, sc1, m1);
        for (int32_t d = 0; d < hd; d++) {
            const int32_t b = d >> 5;
            float a = 0.0f, c = 0.0f;
            for (int32_t k = 0; k < kv_len; k++) {
                const float vsk = vs[(size_t)k * nb + b];
                const float v = (float)vq[(size_t)k * hd + d];
                a = fmaf(sc0[k] * vsk, v, a);
                c = fmaf(sc1[k] * vsk, v, c);
            }
            out0[d] = a;
            out1[d] = c;
        }
        return;
    }
    for (int32_t t = 0; t < kv_len; t++) {
        const float s = dot_q8(hd, q0, kq + (size_t)t * hd, ks + (size_t)t * nb) * scale;
        sc0[t] = s;
        if (s > m0) m0 = s;
    }
    softmax_ref(kv_len, sc0, m0);
    for (int32_t d = 0; d < hd; d++) {
        const int32_t b = d >> 5;
        float a = 0.0f;
        for (int32_t k = 0; k < kv_len; k++)
            a = fmaf(sc0[k] * vs[(size_t)k * nb + b], (float)vq[(size_t)k * hd + d], a);
        out0[d] = a;
    }
}

/* ------------------------------------------------------------------------- */
/* A11: SwiGLU with dead zone, 8-wide path (reference dpuf_engine.c:967-989)  */
/* ------------------------------------------------------------------------- */

float orc_swiglu1(float g, float u, float dz) {
    float ng = fmaxf(-40.0f, fminf(0.0f - g, 40.0f));
    float silu = g / (1.0f + orc_exp_poly(ng));
    float r = silu * u;
    if (dz > 0.0f && !(fabsf(r) >= dz)) r = 0.0f;
    return r;
}

/* ------------------------------------------------------------------------- */
/* A14/A15: engine (reference dpuf_engine.c:1182-2170)                        */
/* ------------------------------------------------------------------------- */

/* fp32 K/V [L][n_kv][max_seq][hd], or with kv_type 1 int8 K/V of that
 * layout plus per-32 scales [L][n_kv][max_seq][hd/32] (dpuf_engine.c:1182-1206). */
typedef struct {
    float* k;
    float* v;
    int8_t* kq;
    int8_t* vq;
    float* ks;
    float* vs;
    int allocated;
} OrcSlot;

typedef struct {
    float* k;
    float* v;
    int8_t* kq;
    int8_t* vq;
    float* ks;
    float* vs;
    int32_t len;
    int valid;
} OrcPrefix;

struct OrcEngine {
    DpufModelConfig cfg;
    DpufLayerWeights* layers;
    DpufWeightDesc tok, lm;
    const float* out_norm;
    float* cos_tab;
    float* sin_tab;
    OrcSlot slots[ORC_MAX_SLOTS];
    OrcPrefix prefixes[ORC_MAX_PREFIXES];
    int32_t active;
    float deadzone;
    float* capture;   /* [num_layers][M][H] residual after each layer, or NULL */
    int32_t capture_cap;
};

static size_t kv_elems(const OrcEngine* e) {
    return (size_t)e->cfg.num_layers * (size_t)e->cfg.max_seq_len *
           (size_t)e->cfg.num_kv_heads * (size_t)e->cfg.head_dim;
}

static int is_q8(const OrcEngine* e) { return e->cfg.kv_type == DPUF_KV_Q8; }

static int slot_alloc(OrcEngine* e, int32_t s) {
    OrcSlot* sl = &e->slots[s];
    if (sl->allocated) return 1;
    if (is_q8(e)) {
        sl->kq = (int8_t*)calloc(kv_elems(e), 1);
        sl->vq = (int8_t*)calloc(kv_elems(e), 1);
        sl->ks = (float*)calloc(kv_elems(e) / 32, sizeof(float));
        sl->vs = (float*)calloc(kv_elems(e) / 32, sizeof(float));
        if (!sl->kq || !sl->vq || !sl->ks || !sl->vs) return 0;
    } else {
        sl->k = (float*)calloc(kv_elems(e), sizeof(float));
        sl->v = (float*)calloc(kv_elems(e), sizeof(float));
        if (!sl->k || !sl->v) return 0;
    }
    sl->allocated = 1;
    return 1;
}

OrcEngine* orc_engine_create(const DpufModelConfig* cfg, const DpufLayerWeights* layers,
                             const DpufWeightDesc* tok, const DpufWeightDesc* lm,
                             const float* out_norm) {
    if (!cfg || !layers || !tok || !lm || !out_norm) return NULL;
    OrcEngine* e = (OrcEngine*)calloc(1, sizeof(OrcEngine));
    e->cfg = *cfg;
    e->layers = (DpufLayerWeights*)malloc((size_t)(cfg->num_layers > 0 ? cfg->num_layers : 1) * sizeof(DpufLayerWeights));
    memcpy(e->layers, layers, (size_t)cfg->num_layers * sizeof(DpufLayerWeights));
    e->tok = *tok;
    e->lm = *lm;
    e->out_norm = out_norm;
    const char* dz = getenv("DPUF_SWIGLU_DEADZONE");
    e->deadzone = dz ? (float)atof(dz) : 0.005f;
    size_t half = (size_t)(cfg->head_dim >> 1);
    e->cos_tab = (float*)malloc((size_t)cfg->max_seq_len * half * sizeof(float));
    e->sin_tab = (float*)malloc((size_t)cfg->max_seq_len * half * sizeof(float));
    orc_rope_tables(&e->cfg, e->cos_tab, e->sin_tab);
    if (!slot_alloc(e, 0)) { orc_engine_destroy(e); return NULL; }
    return e;
}

void orc_engine_destroy(OrcEngine* e) {
    if (!e) return;
    for (int s = 0; s < ORC_MAX_SLOTS; s++) {
        OrcSlot* sl = &e->slots[s];
        free(sl->k); free(sl->v); free(sl->kq); free(sl->vq); free(sl->ks); free(sl->vs);
    }
    for (int p = 0; p < ORC_MAX_PREFIXES; p++) {
        OrcPrefix* pf = &e->prefixes[p];
        free(pf->k); free(pf->v); free(pf->kq); free(pf->vq); free(pf->ks); free(pf->vs);
    }
    free(e->cos_tab); free(e->sin_tab); free(e->layers); free(e->capture);
    free(e);
}

int32_t orc_engine_set_slot(OrcEngine* e, int32_t s) {
    if (!e || s < 0 || s >= ORC_MAX_SLOTS) return -1;
    if (!slot_alloc(e, s)) return -2;
    e->active = s;
    return 0;
}

void orc_engine_reset_slot(OrcEngine* e, int32_t s) {
    if (!e || s < 0 || s >= ORC_MAX_SLOTS || !e->slots[s].allocated) return;
    OrcSlot* sl = &e->slots[s];
    if (is_q8(e)) {
        memset(sl->kq, 0, kv_elems(e));
        memset(sl->vq, 0, kv_elems(e));
        memset(sl->ks, 0, kv_elems(e) / 32 * sizeof(float));
        memset(sl->vs, 0, kv_elems(e) / 32 * sizeof(float));
    } else {
        memset(sl->k, 0, kv_elems(e) * sizeof(float));
        memset(sl->v, 0, kv_elems(e) * sizeof(float));
    }
}

/* Copies positions [0, len) of every (layer, kv head) between a slot's
 * layout [..][max_seq][..] and a prefix's [..][len][..] (to_prefix selects
 * the direction), for each array the cache has. */
static void prefix_copy(OrcEngine* e, OrcSlot* sl, OrcPrefix* p, int32_t len, int to_prefix) {
    const size_t hd = (size_t)e->cfg.head_dim, nkv = (size_t)e->cfg.num_kv_heads, L = (size_t)e->cfg.num_layers;
    const size_t ms = (size_t)e->cfg.max_seq_len;
    for (size_t l = 0; l < L; l++)
        for (size_t h = 0; h < nkv; h++) {
            const size_t po = (l * nkv + h) * (size_t)len, so = (l * nkv + h) * ms;
#define PCOPY(S, P, T, W)                                                                        \
    do {                                                                                           \
        T* dst = to_prefix ? (P) + po * (W) : (S) + so * (W);                                     \
        const T* src = to_prefix ? (S) + so * (W) : (P) + po * (W);                               \
        memcpy(dst, src, (size_t)len * (W) * sizeof(T));                                           \
    } while (0)
            if (is_q8(e)) {
                PCOPY(sl->kq, p->kq, int8_t, hd);
                PCOPY(sl->vq, p->vq, int8_t, hd);
                PCOPY(sl->ks, p->ks, float, hd / 32);
                PCOPY(sl->vs, p->vs, float, hd / 32);
            } else {
                PCOPY(sl->k, p->k, float, hd);
                PCOPY(sl->v, p->v, float, hd);
            }
#undef PCOPY
        }
}

/* Prefix copies follow dpuf_engine.c:1471-1600 (layout [L][kvh][len][hd]). */
int32_t orc_engine_freeze_prefix(OrcEngine* e, int32_t id, int32_t len) {
    if (!e || id < 0 || id >= ORC_MAX_PREFIXES || len <= 0 || len > e->cfg.max_seq_len) return 0;
    OrcPrefix* p = &e->prefixes[id];
    size_t hd = (size_t)e->cfg.head_dim, nkv = (size_t)e->cfg.num_kv_heads, L = (size_t)e->cfg.num_layers;
    const size_t n = L * nkv * (size_t)len * hd;
    free(p->k); free(p->v); free(p->kq); free(p->vq); free(p->ks); free(p->vs);
    memset(p, 0, sizeof *p);
    if (is_q8(e)) {
        p->kq = (int8_t*)calloc(n, 1);
        p->vq = (int8_t*)calloc(n, 1);
        p->ks = (float*)calloc(n / 32, sizeof(float));
        p->vs = (float*)calloc(n / 32, sizeof(float));
    } else {
        p->k = (float*)calloc(n, sizeof(float));
        p->v = (float*)calloc(n, sizeof(float));
    }
    prefix_copy(e, &e->slots[e->active], p, len, 1);
    p->len = len;
    p->valid = 1;
    return 1;
}

int32_t orc_engine_apply_prefix(OrcEngine* e, int32_t slot, int32_t id) {
    if (!e || slot < 0 || slot >= ORC_MAX_SLOTS || id < 0 || id >= ORC_MAX_PREFIXES) return 0;
    OrcPrefix* p = &e->prefixes[id];
    if (!p->valid || p->len <= 0) return 0;
    if (!slot_alloc(e, slot)) return 0;
    prefix_copy(e, &e->slots[slot], p, p->len, 0);
    return p->len;
}

/* Writes positions [pos0, pos0+n) of one (layer, kv head) in the active slot:
 * the KV-inject hook used for the long-context workload. */
int32_t orc_engine_set_kv(OrcEngine* e, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                          const float* k, const float* v) {
    if (!e || layer < 0 || layer >= e->cfg.num_layers || kvh < 0 || kvh >= e->cfg.num_kv_heads ||
        pos0 < 0 || n < 0 || pos0 + n > e->cfg.max_seq_len) return -1;
    OrcSlot* sl = &e->slots[e->active];
    size_t hd = (size_t)e->cfg.head_dim;
    size_t off = (((size_t)layer * e->cfg.num_kv_heads + kvh) * (size_t)e->cfg.max_seq_len + pos0) * hd;
    if (is_q8(e)) {
        /* rows are quantised as the KV store does (dpuf_engine.c:1800-1806) */
        for (int32_t i = 0; i < n; i++) {
            orc_quant_q8((int32_t)hd, k + (size_t)i * hd, sl->kq + off + (size_t)i * hd, sl->ks + (off + (size_t)i * hd) / 32);
            orc_quant_q8((int32_t)hd, v + (size_t)i * hd, sl->vq + off + (size_t)i * hd, sl->vs + (off + (size_t)i * hd) / 32);
        }
        return 0;
    }
    memcpy(sl->k + off, k, (size_t)n * hd * sizeof(float));
    memcpy(sl->v + off, v, (size_t)n * hd * sizeof(float));
    return 0;
}

int32_t orc_engine_get_kv(OrcEngine* e, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                          float* k, float* v) {
    if (!e || layer < 0 || layer >= e->cfg.num_layers || kvh < 0 || kvh >= e->cfg.num_kv_heads ||
        pos0 < 0 || n < 0 || pos0 + n > e->cfg.max_seq_len) return -1;
    OrcSlot* sl = &e->slots[e->active];
    size_t hd = (size_t)e->cfg.head_dim;
    size_t off = (((size_t)layer * e->cfg.num_kv_heads + kvh) * (size_t)e->cfg.max_seq_len + pos0) * hd;
    if (is_q8(e)) { /* dequantised: q * scale */
        for (size_t i = 0; i < (size_t)n * hd; i++) {
            k[i] = (float)sl->kq[off + i] * sl->ks[(off + i) / 32];
            v[i] = (float)sl->vq[off + i] * sl->vs[(off + i) / 32];
        }
        return 0;
    }
    memcpy(k, sl->k + off, (size_t)n * hd * sizeof(float));
    memcpy(v, sl->v + off, (size_t)n * hd * sizeof(float));
    return 0;
}

/* Enables capture of the residual stream after every layer for up to
 * max_tokens rows (0 disables).  Read back with orc_engine_get_capture. */
void orc_engine_set_capture(OrcEngine* e, int32_t max_tokens) {
    free(e->capture);
    e->capture = NULL;
    e->capture_cap = 0;
    if (max_tokens > 0) {
        e->capture = (float*)calloc((size_t)e->cfg.num_layers * max_tokens * e->cfg.hidden_size, sizeof(float));
        e->capture_cap = max_tokens;
    }
}

const float* orc_engine_get_capture(OrcEngine* e) { return e->capture; }

/* Prep + GEMM of one weight for M rows of x, writing out [M][rows]. */
static void run_weight(const DpufWeightDesc* w, int32_t M, const float* x, float* out,
                       int32_t t0, int32_t t1, int8_t* q, float* s, int32_t* m) {
    int32_t cols = w->cols, n_blk = cols >> 5;
    for (int32_t i = 0; i < M; i++)
        orc_prep_row(cols, x + (size_t)i * cols, w->sign_bits, q + (size_t)i * cols,
                     s + (size_t)i * n_blk, m + (size_t)i * n_blk);
    if (w->mode == DPUF_MODE_QR_HAD4_PACKED)
        orc_gemm_tiles(M, w->rows, cols, t0, t1, q, s, m, w->tensor_base, w->tile_offsets, out, M == 1);
    else
        orc_gemm_tiles_asym(w->mode == DPUF_MODE_QR_HAD6, M, w->rows, cols, t0, t1, q, s, m, w->tensor_base,
                            w->tile_offsets, out);
}

int32_t orc_engine_forward(OrcEngine* e, int32_t n_tokens, const int32_t* ids, int32_t pos0,
                           const float* embeds_in, int32_t only_last, float* logits) {
    if (!e || (!ids && !embeds_in) || (!logits && only_last != 2)) return -1;
    if (n_tokens <= 0 || n_tokens > ORC_MAX_BATCH) return -2;
    if (pos0 < 0 || pos0 + n_tokens > e->cfg.max_seq_len) return -3;
    const DpufModelConfig* c = &e->cfg;
    const int32_t M = n_tokens, H = c->hidden_size, I = c->intermediate_size, L = c->num_layers;
    const int32_t nq = c->num_q_heads, nkv = c->num_kv_heads, hd = c->head_dim;
    const int32_t qd = nq * hd, kvd = nkv * hd, groups = nq / nkv, half = hd >> 1;
    const float eps = c->rms_eps;
    const float scale = 1.0f / sqrtf((float)hd);
    int32_t maxd = H > I ? H : I;
    if (qd > maxd) maxd = qd;

    float* h = (float*)calloc((size_t)M * H, sizeof(float));
    float* hn = (float*)calloc((size_t)M * H, sizeof(float));
    float* xn = (float*)calloc((size_t)M * maxd, sizeof(float));
    float* qb = (float*)calloc((size_t)M * qd, sizeof(float));
    float* kb = (float*)calloc((size_t)M * kvd, sizeof(float));
    float* vb = (float*)calloc((size_t)M * kvd, sizeof(float));
    float* ao = (float*)calloc((size_t)M * qd, sizeof(float));
    float* gb = (float*)calloc((size_t)M * I, sizeof(float));
    float* ub = (float*)calloc((size_t)M * I, sizeof(float));
    int8_t* pq = (int8_t*)calloc((size_t)M * maxd, 1);
    float* ps = (float*)calloc((size_t)M * (maxd >> 5), sizeof(float));
    int32_t* pm = (int32_t*)calloc((size_t)M * (maxd >> 5), sizeof(int32_t));

    /* Embedding / embeds_in (dpuf_engine.c:1658-1672). */
    for (int32_t m = 0; m < M; m++) {
        if (embeds_in && (!ids || ids[m] < 0))
            memcpy(h + (size_t)m * H, embeds_in + (size_t)m * H, (size_t)H * sizeof(float));
        else
            orc_embed_desc(&e->tok, 1, ids + m, h + (size_t)m * H);
    }

    OrcSlot* sl = &e->slots[e->active];
    const size_t lstride = (size_t)c->max_seq_len * kvd, hstride = (size_t)c->max_seq_len * hd;

    for (int32_t l = 0; l < L; l++) {
        const DpufLayerWeights* lw = &e->layers[l];
        /* (1) [h += previous down output] + attn RMSNorm. */
        for (int32_t m = 0; m < M; m++)
            orc_add_rmsnorm(H, h + (size_t)m * H, l > 0 ? hn + (size_t)m * H : NULL, lw->attn_norm, eps, xn + (size_t)m * H);
        /* (2) Q, K, V projections. */
        run_weight(&lw->w_q, M, xn, qb, 0, lw->w_q.n_tiles, pq, ps, pm);
        run_weight(&lw->w_k, M, xn, kb, 0, lw->w_k.n_tiles, pq, ps, pm);
        run_weight(&lw->w_v, M, xn, vb, 0, lw->w_v.n_tiles, pq, ps, pm);
        /* (3) K: QK-norm, RoPE, cache store; Q: QK-norm, RoPE (dpuf_engine.c:1791-1817). */
        float* kc = is_q8(e) ? NULL : sl->k + (size_t)l * lstride;
        float* vc = is_q8(e) ? NULL : sl->v + (size_t)l * lstride;
        for (int32_t m = 0; m < M; m++) {
            int32_t pos = pos0 + m;
            const float* cp = e->cos_tab + (size_t)pos * half;
            const float* sp = e->sin_tab + (size_t)pos * half;
            for (int32_t k = 0; k < nkv; k++) {
                float* ks = kb + (size_t)m * kvd + (size_t)k * hd;
                float* vs = vb + (size_t)m * kvd + (size_t)k * hd;
                if (c->has_qk_norm && lw->attn_k_norm) orc_add_rmsnorm(hd, ks, NULL, lw->attn_k_norm, eps, ks);
                orc_rope_apply(hd, ks, cp, sp);
                if (is_q8(e)) {
                    const size_t o = (size_t)l * lstride + (size_t)k * hstride + (size_t)pos * hd;
                    orc_quant_q8(hd, ks, sl->kq + o, sl->ks + o / 32);
                    orc_quant_q8(hd, vs, sl->vq + o, sl->vs + o / 32);
                } else {
                    memcpy(kc + (size_t)k * hstride + (size_t)pos * hd, ks, (size_t)hd * sizeof(float));
                    memcpy(vc + (size_t)k * hstride + (size_t)pos * hd, vs, (size_t)hd * sizeof(float));
                }
            }
            for (int32_t qh = 0; qh < nq; qh++) {
                float* qv = qb + (size_t)m * qd + (size_t)qh * hd;
                if (c->has_qk_norm && lw->attn_q_norm) orc_add_rmsnorm(hd, qv, NULL, lw->attn_q_norm, eps, qv);
                orc_rope_apply(hd, qv, cp, sp);
            }
        }
        /* (3b) causal GQA attention, head pairs. */
        int32_t task;
#pragma omp parallel for schedule(dynamic, 1)
        for (task = 0; task < M * nkv; task++) {
            int32_t m = task / nkv, k = task % nkv;
            int32_t kv_len = pos0 + m + 1;
            float* s0 = (float*)malloc((size_t)kv_len * sizeof(float));
            float* s1 = (float*)malloc((size_t)kv_len * sizeof(float));
            for (int32_t g = 0; g < groups; g += 2) {
                int32_t qh = k * groups + g;
                int has_p = (g + 1 < groups);
                const float* q0 = qb + (size_t)m * qd + (size_t)qh * hd;
                float* a0 = ao + (size_t)m * qd + (size_t)qh * hd;
                if (is_q8(e)) {
                    const size_t o = (size_t)l * lstride + (size_t)k * hstride;
                    orc_attn_heads_q8(hd, kv_len, scale, sl->kq + o, sl->ks + o / 32, sl->vq + o, sl->vs + o / 32,
                                      q0, has_p ? q0 + hd : NULL, s0, s1, a0, has_p ? a0 + hd : NULL);
                } else {
                    orc_attn_heads(hd, kv_len, scale, kc + (size_t)k * hstride, vc + (size_t)k * hstride,
                                   q0, has_p ? q0 + hd : NULL, s0, s1, a0, has_p ? a0 + hd : NULL);
                }
            }
            free(s0); free(s1);
        }
        /* (4) O projection into hn. */
        run_weight(&lw->w_o, M, ao, hn, 0, lw->w_o.n_tiles, pq, ps, pm);
        /* (5) h += O; FFN RMSNorm. */
        for (int32_t m = 0; m < M; m++)
            orc_add_rmsnorm(H, h + (size_t)m * H, hn + (size_t)m * H, lw->ffn_norm, eps, xn + (size_t)m * H);
        /* (6) gate / up; (7) SwiGLU with dead zone. */
        run_weight(&lw->w_gate, M, xn, gb, 0, lw->w_gate.n_tiles, pq, ps, pm);
        run_weight(&lw->w_up, M, xn, ub, 0, lw->w_up.n_tiles, pq, ps, pm);
        for (size_t i = 0; i < (size_t)M * I; i++) gb[i] = orc_swiglu1(gb[i], ub[i], e->deadzone);
        /* (8) down projection, optionally pruned to the first keep tiles
         * with the remaining rows zeroed (dpuf_engine.c:2018-2044). */
        int32_t keep = lw->w_down.n_tiles;
        const char* kt = getenv(M > 1 ? "DPUF_PREFILL_KEEP_TILES" : "DPUF_GEN_KEEP_TILES");
        if (kt) {
            int32_t v = atoi(kt);
            if (v > 0 && v < keep) keep = v;
        }
        run_weight(&lw->w_down, M, gb, hn, 0, keep, pq, ps, pm);
        if (keep < lw->w_down.n_tiles) {
            for (int32_t m = 0; m < M; m++)
                for (int32_t r = keep * 16; r < lw->w_down.rows; r++) hn[(size_t)m * H + r] = 0.0f;
        }
        if (e->capture && M <= e->capture_cap) {
            for (int32_t m = 0; m < M; m++)
                for (int32_t i = 0; i < H; i++)
                    e->capture[((size_t)l * e->capture_cap + m) * H + i] = h[(size_t)m * H + i] + hn[(size_t)m * H + i];
        }
    }

    /* Final residual + output norm + LM head (dpuf_engine.c:2058-2139). */
    if (only_last != 2) {
        int32_t lm0 = only_last ? M - 1 : 0;
        int32_t lmM = M - lm0;
        for (int32_t i = 0; i < lmM; i++) {
            int32_t m = lm0 + i;
            orc_add_rmsnorm(H, h + (size_t)m * H, L > 0 ? hn + (size_t)m * H : NULL, e->out_norm, eps, xn + (size_t)i * H);
        }
        const DpufWeightDesc* w = &e->lm;
        const char* et = getenv("DPUF_EARLY_TILES");
        if (et && lmM == 1 && w->n_tiles > 2048) {
            int32_t za = atoi(et);
            if (za < 256) za = 256;
            if (za > w->n_tiles) za = w->n_tiles;
            run_weight(w, 1, xn, logits, 0, za, pq, ps, pm);
            int32_t nz = za * 16;
            if (nz > c->vocab_size) nz = c->vocab_size;
            const char* em = getenv("DPUF_EARLY_MARGIN");
            float thr = em ? (float)atof(em) : 1.25f;
            if (orc_top2_exit(logits, nz, thr)) {
                for (int32_t i = za * 16; i < c->vocab_size; i++) logits[i] = -1e9f;
            } else {
                /* Prep again and finish the remaining tiles (same values). */
                run_weight(w, 1, xn, logits, za, w->n_tiles, pq, ps, pm);
            }
        } else {
            run_weight(w, lmM, xn, logits, 0, w->n_tiles, pq, ps, pm);
        }
    }

    free(h); free(hn); free(xn); free(qb); free(kb); free(vb); free(ao);
    free(gb); free(ub); free(pq); free(ps); free(pm);
    return 0;
}

/* Zone-A early-exit test of dpuf_engine.c:2101-2110: the sequential top-1 /
 * top-2 scan from -1e30 (a value equal to the top counts as the second), then
 * exit when thr > 0 and top1 - top2 >= thr. */
int32_t orc_top2_exit(const float* x, int32_t n, float thr) {
    float b1 = -1e30f, b2 = -1e30f;
    for (int32_t i = 0; i < n; i++) {
        float v = x[i];
        if (v > b1) { b2 = b1; b1 = v; }
        else if (v > b2) { b2 = v; }
    }
    return (thr > 0.0f && (b1 - b2) >= thr) ? 1 : 0;
}

/* Greedy sampler of dpuf-cli.c:1997-2004: first maximum under strict '>'. */
int32_t orc_argmax(const float* logits, int32_t V) {
    int32_t best = 0;
    float bv = logits[0];
    for (int32_t i = 1; i < V; i++) {
        if (logits[i] > bv) { bv = logits[i]; best = i; }
    }
    return best;
}

int32_t orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Sets the OpenMP threads of the following calls (n >= 1); the CPU baseline
 * times a README-comparable thread count with it. */
void orc_set_num_threads(int32_t n) {
#ifdef _OPENMP
    if (n >= 1) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
