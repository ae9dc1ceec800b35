/*
 * dpuf_tools.c -- deterministic random-init weights, the mode 12 packer, the
 * .dpuf container writer and an mmap reader with tile verify / XOR heal.
 *
 * Format references (all layouts are kept byte-compatible with the reference
 * so that files written here load in dpuf-cli.c and vice versa):
 *   container  : SPECIFICATION.md:11-51, writer dpuf_format.py:2362-2437
 *   QR blob    : finder "<B4sBHIIIIQQQ16x" dpuf_format.py:936-938, assembler
 *                dpuf_format.py:1182-1252
 *   mode 12    : encoder dpuf_format.py:1434-1536, kernel layout
 *                dpuf_avx2.c:2347-2353
 *   RAW_TINY   : dpuf_format.py:137-147
 *   bind/verify: dpuf-cli.c:1646-1756, 1779-1886
 * The random-init generator is this build's own (splitmix64 + Box-Muller),
 * chosen so that every element is a pure function of (seed, name, index).
 */
#define _GNU_SOURCE
#include "dpuf_tools.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------- */
/* CRC32 (poly 0xEDB88320), bit conversions, RNG                              */
/* ------------------------------------------------------------------------- */

static uint32_t crc_tab[256];
static int crc_ready = 0;

static void crc_init(void) {
    if (crc_ready) return;
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
        crc_tab[i] = c;
    }
    crc_ready = 1;
}

static uint32_t crc32_update(uint32_t crc, const uint8_t* p, size_t n) {
    crc = ~crc;
    for (size_t i = 0; i < n; i++) crc = crc_tab[(crc ^ p[i]) & 0xFFu] ^ (crc >> 8);
    return ~crc;
}

DPUF_EXPORT uint16_t dpuf_tools_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                   /* below 2^-14: subnormal */
        float v;
        memcpy(&v, &ax, 4);
        float m = rintf(v * 16777216.0f);
        return (uint16_t)(sign | (uint32_t)m);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

DPUF_EXPORT float dpuf_tools_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu, man = h & 0x3FFu, bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else {
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FFu) << 13);
        }
    } else if (exp == 31) bits = sign | 0x7F800000u | (man << 13);
    else bits = sign | ((exp + 112u) << 23) | (man << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}

static inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

DPUF_EXPORT void dpuf_tools_round_bf16(float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = bf16_to_f32(f32_to_bf16(x[i]));
}

static inline uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t name_seed(uint64_t seed, const char* name) {
    crc_init();
    uint32_t c = crc32_update(0, (const uint8_t*)name, strlen(name));
    return splitmix64(seed ^ ((uint64_t)c << 32) ^ 0x9E3779B9ull);
}

DPUF_EXPORT void dpuf_tools_random_normal(float* out, size_t n, float std, uint64_t seed, const char* name) {
    const uint64_t base = name_seed(seed, name);
    const size_t npair = (n + 1) / 2;
    long long p;
#pragma omp parallel for schedule(static)
    for (p = 0; p < (long long)npair; p++) {
        uint64_t r = splitmix64(base + (uint64_t)p * 0xD1B54A32D192ED03ull);
        /* two 24-bit uniforms in (0, 1] and [0, 1) */
        float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);
        float u2 = (float)((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
        float rad = sqrtf(-2.0f * logf(u1)) * std;
        float th = 6.283185307179586f * u2;
        size_t i = (size_t)p * 2;
        out[i] = rad * cosf(th);
        if (i + 1 < n) out[i + 1] = rad * sinf(th);
    }
}

DPUF_EXPORT void dpuf_tools_sign_bits(uint8_t* out, int32_t cols, uint64_t seed, const char* sign_name) {
    uint64_t s = name_seed(seed, sign_name);
    for (int32_t b = 0; b < cols / 8; b++) out[b] = (uint8_t)(splitmix64(s + (uint64_t)b) >> 56);
}

/* ------------------------------------------------------------------------- */
/* Mode 12 packer                                                             */
/* ------------------------------------------------------------------------- */

/* Orthonormal FWHT-64 with the butterfly order of dpuf_format.py:966-977. */
static void fwht64(float* y) {
    for (int h = 1; h < 64; h <<= 1)
        for (int i = 0; i < 64; i += 2 * h)
            for (int j = i; j < i + h; j++) {
                float a = y[j], b = y[j + h];
                y[j] = a + b;
                y[j + h] = a - b;
            }
    for (int i = 0; i < 64; i++) y[i] *= 0.125f;
}

/* One row: sign, FWHT-64, then per 32-block the MSE scale search over
 * multipliers {0.78, 0.85, 0.92, 1.00} of amax/7.5 (dpuf_format.py:1462-1490).
 * Writes u4 in [0, 15] (q + 8) and fp16 scale bits. */
static void encode_row(const float* w, int32_t cols, const float* signs, uint8_t* u4, uint16_t* sc, float* tmp) {
    for (int32_t c = 0; c < cols; c++) tmp[c] = w[c] * signs[c];
    for (int32_t c = 0; c < cols; c += 64) fwht64(tmp + c);
    static const float mults[4] = {0.78f, 0.85f, 0.92f, 1.00f};
    for (int32_t b = 0; b < cols / 32; b++) {
        const float* v = tmp + 32 * b;
        float amax = 0.0f;
        for (int k = 0; k < 32; k++) { float a = fabsf(v[k]); if (a > amax) amax = a; }
        float base = amax / 7.5f + 1e-12f;
        uint16_t best = dpuf_tools_f32_to_f16(base);
        float best_err = INFINITY;
        for (int mi = 0; mi < 4; mi++) {
            uint16_t cs = dpuf_tools_f32_to_f16(base * mults[mi]);
            float cf = dpuf_tools_f16_to_f32(cs);
            float safe = cf > 0.0f ? cf : 1.0f;
            float err = 0.0f;
            for (int k = 0; k < 32; k++) {
                float q = rintf(v[k] / safe);
                q = q < -8.0f ? -8.0f : (q > 7.0f ? 7.0f : q);
                float d = v[k] - q * cf;
                err += d * d;
            }
            if (err < best_err) { best_err = err; best = cs; }
        }
        sc[b] = best;
        float sf = dpuf_tools_f16_to_f32(best);
        float safe = sf > 0.0f ? sf : 1.0f;
        for (int k = 0; k < 32; k++) {
            float q = rintf(v[k] / safe);
            q = q < -8.0f ? -8.0f : (q > 7.0f ? 7.0f : q);
            u4[32 * b + k] = (uint8_t)((int)q + 8);
        }
    }
}

static size_t pad64(size_t n) { return (64 - (n % 64)) % 64; }

/* One mode 12 group (8 rows from W, rows past n_8 padded): [n_blk][8] fp16
 * scales, then per 32-block four 32-byte chunks, byte c*32 + ri*4 + k holding
 * columns 8c+k (low nibble) and 8c+4+k (high nibble) of row ri
 * (dpuf_format.py:1500-1523). */
static void encode_group_m12(const float* W, int32_t cols, int32_t n_8, const float* signs, uint8_t* grp,
                             float* tmp, uint8_t* u4) {
    const int32_t n_blk = cols / 32;
    uint16_t* sc = (uint16_t*)grp;
    uint16_t* scrow = (uint16_t*)malloc((size_t)n_blk * sizeof(uint16_t));
    for (int ri = 0; ri < 8; ri++) {
        if (ri < n_8) {
            encode_row(W + (size_t)ri * cols, cols, signs, u4 + (size_t)ri * cols, scrow, tmp);
            for (int32_t b = 0; b < n_blk; b++) sc[(size_t)b * 8 + ri] = scrow[b];
        } else {
            /* padding rows: u = 8, scale 0 (dpuf_format.py:1507-1511) */
            memset(u4 + (size_t)ri * cols, 8, (size_t)cols);
            for (int32_t b = 0; b < n_blk; b++) sc[(size_t)b * 8 + ri] = 0;
        }
    }
    free(scrow);
    uint8_t* qg = grp + (size_t)n_blk * 16u;
    for (int32_t b = 0; b < n_blk; b++)
        for (int c = 0; c < 4; c++)
            for (int ri = 0; ri < 8; ri++)
                for (int k = 0; k < 4; k++) {
                    const uint8_t* ur = u4 + (size_t)ri * cols + 32 * b + 8 * c;
                    qg[(size_t)b * 128 + c * 32 + ri * 4 + k] = (uint8_t)((ur[4 + k] << 4) | ur[k]);
                }
}

/* Weighted least-squares asymmetric code of one 64-block v (after sign and
 * FWHT): q in [0, qmax], value m + q * d with fp16 d and m.  The search of
 * dpuf_format.py:1602-1667: for shrink in {0.90, 0.96, 1.00} start from the
 * shrunk min/max range, refine (d, lo) by lsq_iters weighted least-squares
 * fits of the rounded codes (weights (|v| + 1e-6)^w_pow, or 1 when w_pow <=
 * 0), round d and m to fp16, requantise, and keep the candidate of smallest
 * squared error (strict <, so the first of equal errors stays). */
static void encode_blk64_asym(const float* v, int qmax, float w_pow, uint16_t* d_out, uint16_t* m_out, uint8_t* q_out) {
    static const float shrinks[3] = {0.90f, 0.96f, 1.00f};
    float wt[64];
    float wmin = v[0], wmax = v[0];
    for (int k = 0; k < 64; k++) {
        wt[k] = w_pow > 0.0f ? powf(fabsf(v[k]) + 1e-6f, w_pow) : 1.0f;
        wmin = v[k] < wmin ? v[k] : wmin;
        wmax = v[k] > wmax ? v[k] : wmax;
    }
    float best_err = INFINITY;
    uint16_t best_d = 0, best_m = 0;
    uint8_t best_q[64];
    memset(best_q, 0, sizeof best_q);
    for (int si = 0; si < 3; si++) {
        const float mid = 0.5f * (wmin + wmax);
        const float half = 0.5f * (wmax - wmin) * shrinks[si];
        float lo = mid - half;
        float d = half > 1e-12f ? (2.0f * half) / (float)qmax : 0.0f;
        for (int it = 0; it < 2; it++) {
            const float sd = d > 1e-12f ? d : 1.0f;
            float s0 = 0.0f, sq = 0.0f, sq2 = 0.0f, sw = 0.0f, sqw = 0.0f;
            for (int k = 0; k < 64; k++) {
                float q = rintf((v[k] - lo) / sd);
                q = q < 0.0f ? 0.0f : (q > (float)qmax ? (float)qmax : q);
                s0 += wt[k];
                sq += wt[k] * q;
                sq2 += wt[k] * q * q;
                sw += wt[k] * v[k];
                sqw += wt[k] * q * v[k];
            }
            const float det = s0 * sq2 - sq * sq;
            if (det > 1e-12f) {
                const float dn = (s0 * sqw - sq * sw) / det;
                const float ln = (sw - dn * sq) / s0;
                if (dn > 1e-12f) {
                    d = dn;
                    lo = ln;
                }
            }
        }
        const uint16_t m16 = dpuf_tools_f32_to_f16(lo);
        const uint16_t d16 = dpuf_tools_f32_to_f16(d > 0.0f ? d : 0.0f);
        const float m32 = dpuf_tools_f16_to_f32(m16), d32 = dpuf_tools_f16_to_f32(d16);
        const float sdf = d32 > 0.0f ? d32 : 1.0f;
        uint8_t qc[64];
        float err = 0.0f;
        for (int k = 0; k < 64; k++) {
            float q = rintf((v[k] - m32) / sdf);
            q = q < 0.0f ? 0.0f : (q > (float)qmax ? (float)qmax : q);
            qc[k] = d32 > 0.0f ? (uint8_t)q : 0;
            const float e = (m32 + (float)qc[k] * d32) - v[k];
            err += e * e;
        }
        if (err < best_err) {
            best_err = err;
            best_d = d16;
            best_m = m16;
            memcpy(best_q, qc, 64);
        }
    }
    *d_out = best_d;
    *m_out = best_m;
    memcpy(q_out, best_q, 64);
}

/* One mode 13 / 14 group (8 rows, rows past n_8 all zero as in
 * dpuf_format.py:1688-1697): dm [n_64][16] fp16 (d of rows 0..7, then m),
 * q4 [n_blk][128] in the mode 12 nibble interleave of the low 4 bits, and
 * for 6 bits q2 [n_blk][64] with bits 4..5 of row ri, column 32b+8c+4h+k at
 * bits 2(ri>>1) of byte c*16 + h*8 + (ri&1)*4 + k (dpuf_format.py:1699-1718). */
static void encode_group_asym(const float* W, int32_t cols, int32_t n_8, const float* signs, int bits, float w_pow,
                              uint8_t* grp, float* tmp, uint8_t* u) {
    const int32_t n_64 = cols / 64, n_blk = cols / 32;
    const int qmax = (1 << bits) - 1;
    uint16_t* dm = (uint16_t*)grp;
    memset(u, 0, (size_t)8 * cols);
    memset(dm, 0, (size_t)n_64 * 32u);
    for (int ri = 0; ri < n_8; ri++) {
        const float* w = W + (size_t)ri * cols;
        for (int32_t c = 0; c < cols; c++) tmp[c] = w[c] * signs[c];
        for (int32_t c = 0; c < cols; c += 64) fwht64(tmp + c);
        for (int32_t g = 0; g < n_64; g++)
            encode_blk64_asym(tmp + 64 * g, qmax, w_pow, &dm[(size_t)g * 16 + ri], &dm[(size_t)g * 16 + 8 + ri],
                              u + (size_t)ri * cols + 64 * g);
    }
    uint8_t* q4 = grp + (size_t)n_64 * 32u;
    for (int32_t b = 0; b < n_blk; b++)
        for (int c = 0; c < 4; c++)
            for (int ri = 0; ri < 8; ri++)
                for (int k = 0; k < 4; k++) {
                    const uint8_t* ur = u + (size_t)ri * cols + 32 * b + 8 * c;
                    q4[(size_t)b * 128 + c * 32 + ri * 4 + k] = (uint8_t)(((ur[4 + k] & 15) << 4) | (ur[k] & 15));
                }
    if (bits == 6) {
        uint8_t* q2 = q4 + (size_t)n_blk * 128u;
        memset(q2, 0, (size_t)n_blk * 64u);
        for (int32_t b = 0; b < n_blk; b++)
            for (int c = 0; c < 4; c++)
                for (int h = 0; h < 2; h++)
                    for (int ri = 0; ri < 8; ri++)
                        for (int k = 0; k < 4; k++) {
                            const uint8_t hv = (uint8_t)((u[(size_t)ri * cols + 32 * b + 8 * c + 4 * h + k] >> 4) & 3);
                            q2[(size_t)b * 64 + c * 16 + h * 8 + (ri & 1) * 4 + k] |= (uint8_t)(hv << ((ri >> 1) * 2));
                        }
    }
}

/* A QR blob of one matrix (dpuf_format.py:1182-1252 _assemble_qr_blob): the
 * 64-byte finder header "<B4sBHIIIIQQQ16x", tile offsets, ECC offsets, sign
 * bits, the tiles (16-byte header with the body's CRC32 and n_rows, body
 * n_8g * grp_bytes, padded to 64), then per ECC group the XOR parity of its
 * padded tiles.  bits 0 packs mode 12, 4 mode 13, 6 mode 14. */
static uint8_t* pack_qr(const float* W, int32_t rows, int32_t cols, const uint8_t* sign_bits, int32_t ecc_group,
                        int bits, float w_pow, size_t* len) {
    crc_init();
    if (rows <= 0 || cols <= 0 || (cols % 64) != 0 || (bits != 0 && bits != 4 && bits != 6)) return NULL;
    const int32_t n_blk = cols / 32;
    const int32_t n_tiles = (rows + 15) / 16;
    const size_t grp_bytes = (size_t)n_blk * (bits == 6 ? 208u : 144u);
    const uint8_t mode = bits == 0 ? DPUF_MODE_QR_HAD4_PACKED : bits == 4 ? DPUF_MODE_QR_HAD4_ASYM : DPUF_MODE_QR_HAD6;
    /* Every tile but possibly the last holds 2 groups; sizes are padded to 64. */
    size_t* t_off = (size_t*)malloc(((size_t)n_tiles + 1) * sizeof(size_t));
    size_t cur = 0;
    for (int32_t t = 0; t < n_tiles; t++) {
        int32_t n_r = (t * 16 + 16 <= rows) ? 16 : rows - t * 16;
        size_t raw = 16u + (size_t)((n_r + 7) / 8) * grp_bytes;
        t_off[t] = cur;
        cur += raw + pad64(raw);
    }
    t_off[n_tiles] = cur;
    const size_t tiles_total = cur;
    const int32_t n_ecc = ecc_group > 0 ? (n_tiles + ecc_group - 1) / ecc_group : 0;
    size_t* e_off = (size_t*)malloc(((size_t)n_ecc + 1) * sizeof(size_t));
    size_t ecur = 0;
    for (int32_t g = 0; g < n_ecc; g++) {
        int32_t g0 = g * ecc_group, g1 = g0 + ecc_group < n_tiles ? g0 + ecc_group : n_tiles;
        size_t mx = 0;
        for (int32_t t = g0; t < g1; t++) { size_t l = t_off[t + 1] - t_off[t]; if (l > mx) mx = l; }
        e_off[g] = ecur;
        ecur += mx;
    }
    e_off[n_ecc] = ecur;

    const size_t tables = 64u + ((size_t)n_tiles + 1) * 8u + ((size_t)n_ecc + 1) * 8u;
    const size_t aux_off = tables + pad64(tables);
    const size_t after_aux = aux_off + (size_t)cols / 8u;
    const size_t tiles_off = after_aux + pad64(after_aux);
    const size_t ecc_off = tiles_off + tiles_total;
    const size_t total = ecc_off + ecur;
    uint8_t* blob = (uint8_t*)calloc(total, 1);
    if (!blob) { free(t_off); free(e_off); return NULL; }

    uint8_t* h = blob;
    h[0] = mode;
    memcpy(h + 1, "QRDP", 4);
    h[5] = 16;
    uint16_t eg = (uint16_t)ecc_group;
    memcpy(h + 6, &eg, 2);
    uint32_t u32v;
    u32v = (uint32_t)rows; memcpy(h + 8, &u32v, 4);
    u32v = (uint32_t)cols; memcpy(h + 12, &u32v, 4);
    u32v = (uint32_t)n_tiles; memcpy(h + 16, &u32v, 4);
    u32v = (uint32_t)n_ecc; memcpy(h + 20, &u32v, 4);
    uint64_t u64v;
    u64v = aux_off; memcpy(h + 24, &u64v, 8);
    u64v = tiles_off; memcpy(h + 32, &u64v, 8);
    u64v = ecc_off; memcpy(h + 40, &u64v, 8);
    for (int32_t t = 0; t <= n_tiles; t++) { u64v = t_off[t]; memcpy(blob + 64 + (size_t)t * 8, &u64v, 8); }
    for (int32_t g = 0; g <= n_ecc; g++) {
        u64v = e_off[g];
        memcpy(blob + 64 + ((size_t)n_tiles + 1) * 8 + (size_t)g * 8, &u64v, 8);
    }
    memcpy(blob + aux_off, sign_bits, (size_t)cols / 8u);

    float* signs = (float*)malloc((size_t)cols * sizeof(float));
    for (int32_t c = 0; c < cols; c++) signs[c] = ((sign_bits[c >> 3] >> (c & 7)) & 1u) ? -1.0f : 1.0f;

    int32_t t;
#pragma omp parallel for schedule(dynamic, 4)
    for (t = 0; t < n_tiles; t++) {
        float* tmp = (float*)malloc((size_t)cols * sizeof(float));
        uint8_t* u = (uint8_t*)malloc((size_t)cols * 8u);
        int32_t n_r = (t * 16 + 16 <= rows) ? 16 : rows - t * 16;
        int32_t n_8g = (n_r + 7) / 8;
        uint8_t* tile = blob + tiles_off + t_off[t];
        uint8_t* body = tile + 16;
        for (int32_t rg = 0; rg < n_8g; rg++) {
            const int32_t n_8 = n_r - rg * 8 < 8 ? n_r - rg * 8 : 8;
            const float* Wg = W + ((size_t)t * 16 + (size_t)rg * 8) * (size_t)cols;
            uint8_t* grp = body + (size_t)rg * grp_bytes;
            if (bits == 0) encode_group_m12(Wg, cols, n_8, signs, grp, tmp, u);
            else encode_group_asym(Wg, cols, n_8, signs, bits, w_pow, grp, tmp, u);
        }
        size_t body_len = (size_t)n_8g * grp_bytes;
        uint32_t crc = crc32_update(0, body, body_len);
        memcpy(tile, &crc, 4);
        uint16_t nr16 = (uint16_t)n_r;
        memcpy(tile + 4, &nr16, 2);
        free(tmp); free(u);
    }
    free(signs);

    /* XOR parity per ECC group over 8-byte words of the padded tiles. */
    for (int32_t g = 0; g < n_ecc; g++) {
        int32_t g0 = g * ecc_group, g1 = g0 + ecc_group < n_tiles ? g0 + ecc_group : n_tiles;
        uint64_t* acc = (uint64_t*)(blob + ecc_off + e_off[g]);
        for (int32_t tt = g0; tt < g1; tt++) {
            size_t nw = (t_off[tt + 1] - t_off[tt]) / 8u;
            const uint8_t* src = blob + tiles_off + t_off[tt];
            for (size_t k = 0; k < nw; k++) {
                uint64_t w;
                memcpy(&w, src + 8 * k, 8);
                acc[k] ^= w;
            }
        }
    }
    free(t_off); free(e_off);
    *len = total;
    return blob;
}

DPUF_EXPORT uint8_t* dpuf_tools_pack_mode12(const float* W, int32_t rows, int32_t cols,
                                            const uint8_t* sign_bits, int32_t ecc_group, size_t* len) {
    return pack_qr(W, rows, cols, sign_bits, ecc_group, 0, 0.0f, len);
}

DPUF_EXPORT uint8_t* dpuf_tools_pack_asym(const float* W, int32_t rows, int32_t cols, const uint8_t* sign_bits,
                                          int32_t ecc_group, int32_t bits, float w_pow, size_t* len) {
    if (bits != 4 && bits != 6) return NULL;
    return pack_qr(W, rows, cols, sign_bits, ecc_group, bits, w_pow, len);
}

DPUF_EXPORT int32_t dpuf_tools_bind_blob(const uint8_t* blob, size_t len, DpufWeightDesc* out) {
    if (!blob || len < 64 || memcmp(blob + 1, "QRDP", 4) != 0) return -1;
    uint32_t rows, cols, n_tiles;
    uint64_t aux_off, tiles_off;
    memcpy(&rows, blob + 8, 4);
    memcpy(&cols, blob + 12, 4);
    memcpy(&n_tiles, blob + 16, 4);
    memcpy(&aux_off, blob + 24, 8);
    memcpy(&tiles_off, blob + 32, 8);
    memset(out, 0, sizeof(*out));
    out->mode = blob[0];
    out->rows = (int32_t)rows;
    out->cols = (int32_t)cols;
    out->n_tiles = (int32_t)n_tiles;
    out->tensor_base = blob + tiles_off;
    out->tile_offsets = (const uint64_t*)(blob + 64);
    out->col_scale = NULL;
    out->sign_bits = blob + aux_off;
    return 0;
}

DPUF_EXPORT uint8_t* dpuf_tools_pack_raw_tiny(const float* v, int32_t n, size_t* len) {
    size_t total = 10u + (size_t)n * 2u;
    uint8_t* b = (uint8_t*)calloc(total, 1);
    b[0] = 0;
    b[1] = 1;
    uint32_t d0 = (uint32_t)n, d1 = 1;
    memcpy(b + 2, &d0, 4);
    memcpy(b + 6, &d1, 4);
    for (int32_t i = 0; i < n; i++) {
        uint16_t x = f32_to_bf16(v[i]);
        memcpy(b + 10 + 2 * (size_t)i, &x, 2);
    }
    *len = total;
    return b;
}

/* ------------------------------------------------------------------------- */
/* Model container                                                            */
/* ------------------------------------------------------------------------- */

typedef struct {
    char* name;
    uint8_t* data;      /* owned blob (built models) or pointer into the map */
    size_t len;
    int owned;
} NamedBlob;

struct DpufToolsModel {
    DpufModelConfig cfg;
    DpufLayerWeights* layers;
    DpufWeightDesc tok, lm;
    float* out_norm;
    int tied;
    NamedBlob* blobs;
    int32_t n_blobs, cap_blobs;
    float** owned_f;     /* fp32 norm copies */
    int32_t n_owned_f, cap_owned_f;
    uint8_t* map_base;
    size_t map_size;
    int32_t healed;
};

static void add_blob(DpufToolsModel* m, const char* name, uint8_t* data, size_t len, int owned) {
    if (m->n_blobs == m->cap_blobs) {
        m->cap_blobs = m->cap_blobs ? m->cap_blobs * 2 : 64;
        m->blobs = (NamedBlob*)realloc(m->blobs, (size_t)m->cap_blobs * sizeof(NamedBlob));
    }
    NamedBlob* nb = &m->blobs[m->n_blobs++];
    nb->name = strdup(name);
    nb->data = data;
    nb->len = len;
    nb->owned = owned;
}

static float* own_floats(DpufToolsModel* m, size_t n) {
    if (m->n_owned_f == m->cap_owned_f) {
        m->cap_owned_f = m->cap_owned_f ? m->cap_owned_f * 2 : 64;
        m->owned_f = (float**)realloc(m->owned_f, (size_t)m->cap_owned_f * sizeof(float*));
    }
    float* p = (float*)malloc(n * sizeof(float));
    m->owned_f[m->n_owned_f++] = p;
    return p;
}

static const NamedBlob* find_blob(const DpufToolsModel* m, const char* name) {
    for (int32_t i = 0; i < m->n_blobs; i++)
        if (strcmp(m->blobs[i].name, name) == 0) return &m->blobs[i];
    return NULL;
}

/* Mode of a matrix under the had4p-hybrid plan (pack_dpuf.py:249-266): 6 bits
 * for ffn_down, attn_v, attn_k, the even layers' attn_output and
 * output.weight, 4 bits for the rest, token_embd included. */
static int hybrid_bits(const char* name) {
    const size_t n = strlen(name);
#define ENDS(sfx) (n >= strlen(sfx) && strcmp(name + n - strlen(sfx), sfx) == 0)
    if (ENDS(".ffn_down.weight") || ENDS(".attn_v.weight") || ENDS(".attn_k.weight") ||
        strcmp(name, "output.weight") == 0)
        return 6;
    if (ENDS(".attn_output.weight") && strncmp(name, "blk.", 4) == 0 && atoi(name + 4) % 2 == 0) return 6;
#undef ENDS
    return 4;
}

/* Tensor names of pack_dpuf.py:122-151.  Plan 0: mode 12 with the sign
 * sharing of pack_dpuf.py:206-216 (sign_name).  Plan 1: the had4p-hybrid
 * plan, each matrix with signs of its own name (pack_dpuf.py:262-264). */
static void build_matrix(DpufToolsModel* m, const DpufToolsSpec* s, const char* name, const char* sign_name,
                         int32_t rows, int32_t cols) {
    float* W = (float*)malloc((size_t)rows * (size_t)cols * sizeof(float));
    dpuf_tools_random_normal(W, (size_t)rows * (size_t)cols, s->weight_std, s->seed, name);
    dpuf_tools_round_bf16(W, (size_t)rows * (size_t)cols);
    uint8_t* sb = (uint8_t*)malloc((size_t)cols / 8u);
    dpuf_tools_sign_bits(sb, cols, s->seed, s->weight_plan == 1 ? name : sign_name);
    size_t len = 0;
    uint8_t* blob = s->weight_plan == 1 ? dpuf_tools_pack_asym(W, rows, cols, sb, 64, hybrid_bits(name), 0.0f, &len)
                                        : dpuf_tools_pack_mode12(W, rows, cols, sb, 64, &len);
    free(W);
    free(sb);
    add_blob(m, name, blob, len, 1);
}

static void build_norm(DpufToolsModel* m, const char* name, int32_t n) {
    float* ones = (float*)malloc((size_t)n * sizeof(float));
    for (int32_t i = 0; i < n; i++) ones[i] = 1.0f;
    size_t len = 0;
    uint8_t* b = dpuf_tools_pack_raw_tiny(ones, n, &len);
    free(ones);
    add_blob(m, name, b, len, 1);
}

/* RAW_TINY -> fp32 heap copy (dpuf-cli.c:1622-1644); NULL unless it holds
 * exactly `want` values (the consumers read that many). */
static float* bind_norm(DpufToolsModel* m, const char* name, int32_t want) {
    const NamedBlob* b = find_blob(m, name);
    if (!b || b->len < 10 || b->data[0] != 0 || want <= 0) return NULL;
    uint32_t d0, d1;
    memcpy(&d0, b->data + 2, 4);
    memcpy(&d1, b->data + 6, 4);
    size_t raw = b->len - 10u;
    if (d1 == 2 && raw == (size_t)d0 * 4u) {
        if (d0 != (uint32_t)want) return NULL;
        float* f = own_floats(m, d0);
        memcpy(f, b->data + 10, raw);
        return f;
    }
    size_t n = raw / 2u;
    if (n != (size_t)want) return NULL;
    float* f = own_floats(m, n);
    for (size_t i = 0; i < n; i++) {
        uint16_t x;
        memcpy(&x, b->data + 10 + 2 * i, 2);
        f[i] = bf16_to_f32(x);
    }
    return f;
}

static int verify_and_heal(DpufToolsModel* m, NamedBlob* nb);

/* Rows of tile t of a matrix of `rows` rows (16 per tile, the last one the
 * remainder) and the body bytes a mode 12 / 13 / 14 tile of n_r rows holds
 * after its 16-byte header. */
static uint32_t tile_rows(uint32_t rows, uint32_t t) { return rows - 16u * t < 16u ? rows - 16u * t : 16u; }
static uint64_t tile_body(uint8_t mode, uint32_t n_r, uint32_t cols) {
    const uint64_t n_8g = (n_r + 7u) / 8u;
    return mode == DPUF_MODE_QR_HAD4_PACKED ? n_8g * (cols / 32u) * 144u
         : mode == DPUF_MODE_QR_HAD4_ASYM   ? n_8g * (cols / 64u) * 288u
                                            : n_8g * (cols / 64u) * 416u;
}

/* The structure of a QR blob against its length, before anything reads
 * through its tables (a file's bytes are untrusted: a damaged count or offset
 * is refused, never followed): mode 12 / 13 / 14, the row / column / tile /
 * ECC-group counts consistent, the tile and ECC offset tables, the sign bytes,
 * the tile region and the ECC region inside the blob, every tile long enough
 * for the body its place in the matrix holds, every ECC block as long as the
 * longest tile of its group.  Tile headers are not checked here: a damaged
 * header is a bad tile for the verify / heal step. */
static int qr_blob_ok(const uint8_t* b, size_t len) {
    if (!b || len < 64 || memcmp(b + 1, "QRDP", 4) != 0) return 0;
    const uint8_t mode = b[0];
    if (mode != DPUF_MODE_QR_HAD4_PACKED && mode != DPUF_MODE_QR_HAD4_ASYM && mode != DPUF_MODE_QR_HAD6) return 0;
    uint16_t G;
    uint32_t rows, cols, n_tiles, n_ecc;
    uint64_t aux_off, tiles_off, ecc_off;
    memcpy(&G, b + 6, 2);
    memcpy(&rows, b + 8, 4);
    memcpy(&cols, b + 12, 4);
    memcpy(&n_tiles, b + 16, 4);
    memcpy(&n_ecc, b + 20, 4);
    memcpy(&aux_off, b + 24, 8);
    memcpy(&tiles_off, b + 32, 8);
    memcpy(&ecc_off, b + 40, 8);
    if (rows == 0 || rows > (1u << 26) || cols == 0 || cols > (1u << 20) || cols % 64u) return 0;
    if (n_tiles != (rows + 15u) / 16u) return 0;
    if (G ? n_ecc != (n_tiles + G - 1u) / G : n_ecc != 0) return 0;
    const uint64_t tables = 64u + ((uint64_t)n_tiles + 1u) * 8u + ((uint64_t)n_ecc + 1u) * 8u;
    if (tables > len || aux_off > len || cols / 8u > len - aux_off) return 0;
    if (tiles_off > ecc_off || ecc_off > len) return 0;
    const uint8_t* to = b + 64;
    const uint8_t* eo = b + 64 + ((size_t)n_tiles + 1u) * 8u;
    uint64_t prev = 0;
    for (uint32_t t = 0; t <= n_tiles; t++) {
        uint64_t o;
        memcpy(&o, to + (size_t)t * 8u, 8);
        if (o < prev || o > ecc_off - tiles_off) return 0;
        if (t > 0 && o - prev < 16u + tile_body(mode, tile_rows(rows, t - 1u), cols)) return 0;
        prev = o;
    }
    uint64_t eprev = 0;
    for (uint32_t g = 0; g <= n_ecc; g++) {
        uint64_t o;
        memcpy(&o, eo + (size_t)g * 8u, 8);
        if (o < eprev || o > len - ecc_off) return 0;
        if (g > 0) {
            const uint32_t g0 = (g - 1u) * G, g1 = g0 + G < n_tiles ? g0 + G : n_tiles;
            for (uint32_t t = g0; t < g1; t++) {
                uint64_t a, z;
                memcpy(&a, to + (size_t)t * 8u, 8);
                memcpy(&z, to + ((size_t)t + 1u) * 8u, 8);
                if (z - a > o - eprev) return 0;
            }
        }
        eprev = o;
    }
    return 1;
}

/* dpuf_qr_verify_tiles_ex over the tiles of a blob that passed qr_blob_ok:
 * a tile whose header claims another row count than its place in the matrix
 * holds is bad without a CRC (the CRC length comes from the header, and
 * would run past the tile); the others are checked as usual.  Returns the
 * number of bad tiles, ok[t] per tile. */
static int32_t verify_tiles_bounded(uint8_t mode, uint32_t rows, uint32_t cols, uint32_t n_tiles,
                                    const uint8_t* tiles, const uint64_t* t_offs, uint8_t* ok) {
    int sane = 1;
    for (uint32_t t = 0; t < n_tiles && sane; t++) {
        DpufQrTileHdr h;
        memcpy(&h, tiles + t_offs[t], sizeof h);
        sane = h.n_rows == tile_rows(rows, t);
    }
    if (sane) return dpuf_qr_verify_tiles_ex(mode, (int32_t)n_tiles, (int32_t)cols, tiles, t_offs, ok);
    int32_t bad = 0;
    for (uint32_t t = 0; t < n_tiles; t++) {
        DpufQrTileHdr h;
        memcpy(&h, tiles + t_offs[t], sizeof h);
        if (h.n_rows != tile_rows(rows, t)) ok[t] = 0;
        else dpuf_qr_verify_tiles_ex(mode, 1, (int32_t)cols, tiles, t_offs + t, ok + t);
        bad += ok[t] ? 0 : 1;
    }
    return bad;
}

static int bind_weight(DpufToolsModel* m, const char* name, int verify, DpufWeightDesc* out) {
    NamedBlob* b = (NamedBlob*)find_blob(m, name);
    if (!b || !qr_blob_ok(b->data, b->len)) return 0;
    if (verify && !verify_and_heal(m, b)) return 0;
    return dpuf_tools_bind_blob(b->data, b->len, out) == 0;
}

static int bind_all(DpufToolsModel* m, int verify) {
    if (!bind_weight(m, "token_embd.weight", verify, &m->tok)) return 0;
    if (!m->tied && find_blob(m, "output.weight")) {
        if (!bind_weight(m, "output.weight", verify, &m->lm)) return 0;
    } else {
        m->lm = m->tok;
    }
    /* every tensor has the shape the configuration gives it: consumers index
     * them by the configuration alone */
    const DpufModelConfig* c = &m->cfg;
    const int32_t H = c->hidden_size, hd = c->head_dim, qd = c->num_q_heads * hd, kvd = c->num_kv_heads * hd;
    if (m->tok.rows != c->vocab_size || m->tok.cols != H || m->lm.rows != c->vocab_size || m->lm.cols != H) return 0;
    m->out_norm = bind_norm(m, "output_norm.weight", H);
    if (!m->out_norm) return 0;
    m->layers = (DpufLayerWeights*)calloc((size_t)(m->cfg.num_layers > 0 ? m->cfg.num_layers : 1), sizeof(DpufLayerWeights));
    char n[96];
    static const char* mats[7] = {"attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down"};
    for (int32_t l = 0; l < m->cfg.num_layers; l++) {
        DpufLayerWeights* lw = &m->layers[l];
        snprintf(n, sizeof n, "blk.%d.attn_norm.weight", l); lw->attn_norm = bind_norm(m, n, H);
        snprintf(n, sizeof n, "blk.%d.ffn_norm.weight", l); lw->ffn_norm = bind_norm(m, n, H);
        if (!lw->attn_norm || !lw->ffn_norm) return 0;
        if (m->cfg.has_qk_norm) {
            snprintf(n, sizeof n, "blk.%d.attn_q_norm.weight", l); lw->attn_q_norm = bind_norm(m, n, hd);
            snprintf(n, sizeof n, "blk.%d.attn_k_norm.weight", l); lw->attn_k_norm = bind_norm(m, n, hd);
            if (!lw->attn_q_norm || !lw->attn_k_norm) return 0;
        }
        DpufWeightDesc* ds[7] = {&lw->w_q, &lw->w_k, &lw->w_v, &lw->w_o, &lw->w_gate, &lw->w_up, &lw->w_down};
        const int32_t want_r[7] = {qd, kvd, kvd, H, c->intermediate_size, c->intermediate_size, H};
        const int32_t want_c[7] = {H, H, H, qd, H, H, c->intermediate_size};
        for (int k = 0; k < 7; k++) {
            snprintf(n, sizeof n, "blk.%d.%s.weight", l, mats[k]);
            if (!bind_weight(m, n, verify, ds[k])) return 0;
            if (ds[k]->rows != want_r[k] || ds[k]->cols != want_c[k]) return 0;
        }
    }
    return 1;
}

static void fill_cfg(DpufModelConfig* c, const DpufToolsSpec* s) {
    memset(c, 0, sizeof(*c));
    c->hidden_size = s->hidden_size;
    c->intermediate_size = s->intermediate_size;
    c->num_layers = s->num_layers;
    c->num_q_heads = s->num_q_heads;
    c->num_kv_heads = s->num_kv_heads;
    c->head_dim = s->head_dim;
    c->vocab_size = s->vocab_size;
    c->max_seq_len = s->max_seq_len;
    c->has_qk_norm = 1;
    c->rms_eps = s->rms_eps;
    c->rope_theta = s->rope_theta;
    c->n_threads = 8;
}

DPUF_EXPORT DpufToolsModel* dpuf_tools_build_model(const DpufToolsSpec* s) {
    DpufToolsModel* m = (DpufToolsModel*)calloc(1, sizeof(DpufToolsModel));
    fill_cfg(&m->cfg, s);
    m->tied = s->tie_word_embeddings;
    const int32_t H = s->hidden_size, I = s->intermediate_size, hd = s->head_dim;
    const int32_t qd = s->num_q_heads * hd, kvd = s->num_kv_heads * hd;
    build_matrix(m, s, "token_embd.weight", "token_embd.weight", s->vocab_size, H);
    if (!m->tied) build_matrix(m, s, "output.weight", "output.weight", s->vocab_size, H);
    build_norm(m, "output_norm.weight", H);
    char n[96], sn[96];
    for (int32_t l = 0; l < s->num_layers; l++) {
        snprintf(n, sizeof n, "blk.%d.attn_norm.weight", l); build_norm(m, n, H);
        snprintf(n, sizeof n, "blk.%d.ffn_norm.weight", l); build_norm(m, n, H);
        snprintf(n, sizeof n, "blk.%d.attn_q_norm.weight", l); build_norm(m, n, hd);
        snprintf(n, sizeof n, "blk.%d.attn_k_norm.weight", l); build_norm(m, n, hd);
        snprintf(sn, sizeof sn, "blk.%d.qkv_in", l);
        snprintf(n, sizeof n, "blk.%d.attn_q.weight", l); build_matrix(m, s, n, sn, qd, H);
        snprintf(n, sizeof n, "blk.%d.attn_k.weight", l); build_matrix(m, s, n, sn, kvd, H);
        snprintf(n, sizeof n, "blk.%d.attn_v.weight", l); build_matrix(m, s, n, sn, kvd, H);
        snprintf(n, sizeof n, "blk.%d.attn_output.weight", l); build_matrix(m, s, n, n, H, qd);
        snprintf(sn, sizeof sn, "blk.%d.mlp_in", l);
        snprintf(n, sizeof n, "blk.%d.ffn_gate.weight", l); build_matrix(m, s, n, sn, I, H);
        snprintf(n, sizeof n, "blk.%d.ffn_up.weight", l); build_matrix(m, s, n, sn, I, H);
        snprintf(n, sizeof n, "blk.%d.ffn_down.weight", l); build_matrix(m, s, n, n, H, I);
    }
    if (!bind_all(m, 0)) { dpuf_tools_free_model(m); return NULL; }
    return m;
}

/* ---- JSON writer / reader (only what the container header needs) -------- */

typedef struct { char* p; size_t n, cap; } Buf;

static void bput(Buf* b, const char* s, size_t n) {
    if (b->n + n + 1 > b->cap) {
        b->cap = (b->n + n + 1) * 2;
        b->p = (char*)realloc(b->p, b->cap);
    }
    memcpy(b->p + b->n, s, n);
    b->n += n;
    b->p[b->n] = 0;
}

static void bprintf(Buf* b, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
#include <stdarg.h>
static void bprintf(Buf* b, const char* fmt, ...) {
    char tmp[512];
    va_list ap;
    va_start(ap, fmt);
    int k = vsnprintf(tmp, sizeof tmp, fmt, ap);
    va_end(ap);
    bput(b, tmp, (size_t)k);
}

DPUF_EXPORT uint64_t dpuf_tools_save_container(const DpufToolsModel* m, const char* path) {
    crc_init();
    /* payload layout: each blob 64-aligned (pack_dpuf.py:370-376) */
    uint64_t* offs = (uint64_t*)malloc((size_t)m->n_blobs * sizeof(uint64_t));
    uint64_t off = 0;
    for (int32_t i = 0; i < m->n_blobs; i++) {
        off += pad64(off);
        offs[i] = off;
        off += m->blobs[i].len;
    }
    const uint64_t payload = off;
    const DpufModelConfig* c = &m->cfg;
    Buf j = {0};
    bprintf(&j, "{\"__metadata__\":{\"format\":\"DPUF / LR-FLAC v1.2.0\",\"format_version\":\"1.2.0\","
                "\"min_reader_version\":\"1.2.0\",\"model_name\":\"random-init\",\"num_tensors\":%d,"
                "\"payload_bytes\":%llu,\"model_config\":{", m->n_blobs, (unsigned long long)payload);
    bprintf(&j, "\"hidden_size\":%d,\"intermediate_size\":%d,\"num_layers\":%d,\"num_q_heads\":%d,"
                "\"num_kv_heads\":%d,\"head_dim\":%d,\"vocab_size\":%d,\"max_seq_len\":%d,",
            c->hidden_size, c->intermediate_size, c->num_layers, c->num_q_heads, c->num_kv_heads,
            c->head_dim, c->vocab_size, c->max_seq_len);
    bprintf(&j, "\"has_qk_norm\":%s,\"rms_eps\":%.9g,\"rope_theta\":%.9g,\"tie_word_embeddings\":%s},"
                "\"tokenizer\":{}},\"__tensors__\":{",
            c->has_qk_norm ? "true" : "false", (double)c->rms_eps, (double)c->rope_theta, m->tied ? "true" : "false");
    for (int32_t i = 0; i < m->n_blobs; i++)
        bprintf(&j, "%s\"%s\":[%llu,%llu]", i ? "," : "", m->blobs[i].name,
                (unsigned long long)offs[i], (unsigned long long)m->blobs[i].len);
    bput(&j, "}}", 2);
    size_t ph = pad64(24u + j.n);
    for (size_t k = 0; k < ph; k++) bput(&j, " ", 1);

    uint32_t pay_crc = 0;
    static const uint8_t zeros[64] = {0};
    uint64_t pos = 0;
    for (int32_t i = 0; i < m->n_blobs; i++) {
        if (offs[i] > pos) pay_crc = crc32_update(pay_crc, zeros, (size_t)(offs[i] - pos));
        pay_crc = crc32_update(pay_crc, m->blobs[i].data, m->blobs[i].len);
        pos = offs[i] + m->blobs[i].len;
    }
    uint32_t hdr_crc = crc32_update(0, (const uint8_t*)j.p, j.n);
    FILE* f = fopen(path, "wb");
    if (!f) { free(offs); free(j.p); return 0; }
    uint8_t top[24];
    memcpy(top, "DPUF0001", 8);
    uint32_t v = (uint32_t)m->n_blobs; memcpy(top + 8, &v, 4);
    memcpy(top + 12, &hdr_crc, 4);
    memcpy(top + 16, &pay_crc, 4);
    v = (uint32_t)j.n; memcpy(top + 20, &v, 4);
    fwrite(top, 1, 24, f);
    fwrite(j.p, 1, j.n, f);
    pos = 0;
    for (int32_t i = 0; i < m->n_blobs; i++) {
        if (offs[i] > pos) fwrite(zeros, 1, (size_t)(offs[i] - pos), f);
        fwrite(m->blobs[i].data, 1, m->blobs[i].len, f);
        pos = offs[i] + m->blobs[i].len;
    }
    fclose(f);
    free(offs);
    uint64_t total = 24u + j.n + payload;
    free(j.p);
    return total;
}

typedef struct { const char* p; const char* e; } Cur;

static void ws(Cur* c) { while (c->p < c->e && (*c->p == ' ' || *c->p == '\n' || *c->p == '\t' || *c->p == '\r')) c->p++; }
static int eat(Cur* c, char ch) { ws(c); if (c->p < c->e && *c->p == ch) { c->p++; return 1; } return 0; }
static int peek(Cur* c) { ws(c); return c->p < c->e ? *c->p : 0; }

static int parse_str(Cur* c, char* out, size_t cap) {
    if (!eat(c, '"')) return 0;
    size_t n = 0;
    while (c->p < c->e && *c->p != '"') {
        char ch = *c->p++;
        if (ch == '\\' && c->p < c->e) ch = *c->p++;
        if (n + 1 < cap) out[n++] = ch;
    }
    if (c->p >= c->e) return 0;
    c->p++;
    out[n] = 0;
    return 1;
}

static int parse_num(Cur* c, double* v) {
    ws(c);
    char* end = NULL;
    *v = strtod(c->p, &end);
    if (end == c->p) return 0;
    c->p = end;
    return 1;
}

static int skip_val(Cur* c) {
    int ch = peek(c);
    char tmp[256];
    double d;
    if (ch == '"') return parse_str(c, tmp, sizeof tmp);
    if (ch == '{' || ch == '[') {
        char open = (char)ch, close = ch == '{' ? '}' : ']';
        eat(c, open);
        if (eat(c, close)) return 1;
        for (;;) {
            if (open == '{') { if (!parse_str(c, tmp, sizeof tmp) || !eat(c, ':')) return 0; }
            if (!skip_val(c)) return 0;
            if (eat(c, ',')) continue;
            return eat(c, close);
        }
    }
    if (!strncmp(c->p, "true", 4)) { c->p += 4; return 1; }
    if (!strncmp(c->p, "false", 5)) { c->p += 5; return 1; }
    if (!strncmp(c->p, "null", 4)) { c->p += 4; return 1; }
    return parse_num(c, &d);
}

static int parse_bool(Cur* c, int* b) {
    ws(c);
    if (!strncmp(c->p, "true", 4)) { c->p += 4; *b = 1; return 1; }
    if (!strncmp(c->p, "false", 5)) { c->p += 5; *b = 0; return 1; }
    return 0;
}

/* Keys of dpuf-cli.c:1199-1237 that this build uses. */
static int parse_cfg(Cur* c, DpufModelConfig* cfg, int* tied) {
    char k[128];
    if (!eat(c, '{')) return 0;
    if (eat(c, '}')) return 1;
    for (;;) {
        if (!parse_str(c, k, sizeof k) || !eat(c, ':')) return 0;
        double d;
        int b;
        if (!strcmp(k, "hidden_size") && parse_num(c, &d)) cfg->hidden_size = (int32_t)d;
        else if (!strcmp(k, "intermediate_size") && parse_num(c, &d)) cfg->intermediate_size = (int32_t)d;
        else if (!strcmp(k, "num_layers") && parse_num(c, &d)) cfg->num_layers = (int32_t)d;
        else if (!strcmp(k, "num_q_heads") && parse_num(c, &d)) cfg->num_q_heads = (int32_t)d;
        else if (!strcmp(k, "num_kv_heads") && parse_num(c, &d)) cfg->num_kv_heads = (int32_t)d;
        else if (!strcmp(k, "head_dim") && parse_num(c, &d)) cfg->head_dim = (int32_t)d;
        else if (!strcmp(k, "vocab_size") && parse_num(c, &d)) cfg->vocab_size = (int32_t)d;
        else if (!strcmp(k, "max_seq_len") && parse_num(c, &d)) cfg->max_seq_len = (int32_t)d;
        else if (!strcmp(k, "has_qk_norm") && parse_bool(c, &b)) cfg->has_qk_norm = b;
        else if (!strcmp(k, "rms_eps") && parse_num(c, &d)) cfg->rms_eps = (float)d;
        else if (!strcmp(k, "rope_theta") && parse_num(c, &d)) cfg->rope_theta = (float)d;
        else if (!strcmp(k, "tie_word_embeddings") && parse_bool(c, &b)) *tied = b;
        else if (!skip_val(c)) return 0;
        if (eat(c, ',')) continue;
        return eat(c, '}');
    }
}

static int parse_header(DpufToolsModel* m, const char* js, size_t n, uint64_t payload_base) {
    Cur c = {js, js + n};
    char k[256];
    int got_cfg = 0, got_tok = 0, got_ten = 0;
    if (!eat(&c, '{')) return 0;
    if (eat(&c, '}')) return 0;
    for (;;) {
        if (!parse_str(&c, k, sizeof k) || !eat(&c, ':')) return 0;
        if (!strcmp(k, "__metadata__")) {
            if (!eat(&c, '{')) return 0;
            if (!eat(&c, '}')) {
                for (;;) {
                    if (!parse_str(&c, k, sizeof k) || !eat(&c, ':')) return 0;
                    if (!strcmp(k, "model_config")) { if (!parse_cfg(&c, &m->cfg, &m->tied)) return 0; got_cfg = 1; }
                    else if (!strcmp(k, "tokenizer")) { if (!skip_val(&c)) return 0; got_tok = 1; }
                    else if (!skip_val(&c)) return 0;
                    if (eat(&c, ',')) continue;
                    if (eat(&c, '}')) break;
                    return 0;
                }
            }
        } else if (!strcmp(k, "__tensors__")) {
            if (!eat(&c, '{')) return 0;
            if (!eat(&c, '}')) {
                for (;;) {
                    double o, l;
                    if (!parse_str(&c, k, sizeof k) || !eat(&c, ':') || !eat(&c, '[') || !parse_num(&c, &o) ||
                        !eat(&c, ',') || !parse_num(&c, &l) || !eat(&c, ']')) return 0;
                    uint64_t off = (uint64_t)o, len = (uint64_t)l;
                    if (payload_base + off + len > m->map_size) return 0;
                    add_blob(m, k, m->map_base + payload_base + off, (size_t)len, 0);
                    if (eat(&c, ',')) continue;
                    if (eat(&c, '}')) break;
                    return 0;
                }
            }
            got_ten = 1;
        } else if (!skip_val(&c)) return 0;
        if (eat(&c, ',')) continue;
        if (eat(&c, '}')) break;
        return 0;
    }
    return got_cfg && got_tok && got_ten;
}

/* Tile CRC check + single-tile XOR heal per ECC group into a heap copy
 * (dpuf-cli.c:1669-1731). */
static int verify_and_heal(DpufToolsModel* m, NamedBlob* nb) {
    const uint8_t* blob = nb->data;
    uint16_t G;
    uint32_t cols, n_tiles, n_ecc;
    uint64_t tiles_off, ecc_off;
    memcpy(&G, blob + 6, 2);
    memcpy(&cols, blob + 12, 4);
    memcpy(&n_tiles, blob + 16, 4);
    memcpy(&n_ecc, blob + 20, 4);
    memcpy(&tiles_off, blob + 32, 8);
    memcpy(&ecc_off, blob + 40, 8);
    uint32_t rows;
    memcpy(&rows, blob + 8, 4);
    const uint64_t* t_offs = (const uint64_t*)(blob + 64);
    const uint64_t* e_offs = (const uint64_t*)(blob + 64 + ((size_t)n_tiles + 1) * 8u);
    uint8_t* ok = (uint8_t*)malloc(n_tiles ? n_tiles : 1);
    int32_t bad = verify_tiles_bounded(blob[0], rows, cols, n_tiles, blob + tiles_off, t_offs, ok);
    if (bad == 0) { free(ok); return 1; }
    if (G == 0) { free(ok); return 0; }
    uint8_t* rw = (uint8_t*)malloc(nb->len);
    memcpy(rw, blob, nb->len);
    uint8_t* wt = rw + tiles_off;
    const uint8_t* we = rw + ecc_off;
    for (uint32_t g = 0; g < n_ecc; g++) {
        uint32_t g0 = g * G, g1 = g0 + G < n_tiles ? g0 + G : n_tiles;
        int nbad = 0;
        uint32_t target = 0;
        for (uint32_t t = g0; t < g1; t++) if (!ok[t]) { target = t; nbad++; }
        if (nbad == 0) continue;
        if (nbad > 1) { free(ok); free(rw); return 0; }
        size_t tlen = (size_t)(t_offs[target + 1] - t_offs[target]);
        uint8_t* dst = wt + t_offs[target];
        memcpy(dst, we + e_offs[g], tlen);
        for (uint32_t p = g0; p < g1; p++) {
            if (p == target) continue;
            size_t plen = (size_t)(t_offs[p + 1] - t_offs[p]);
            size_t nw = (plen < tlen ? plen : tlen) / 8u;
            for (size_t k = 0; k < nw; k++) {
                uint64_t a, b;
                memcpy(&a, dst + 8 * k, 8);
                memcpy(&b, wt + t_offs[p] + 8 * k, 8);
                a ^= b;
                memcpy(dst + 8 * k, &a, 8);
            }
        }
        m->healed++;
    }
    int32_t bad2 = verify_tiles_bounded(blob[0], rows, cols, n_tiles, wt, t_offs, ok);
    free(ok);
    if (bad2 > 0) { free(rw); return 0; }
    nb->data = rw;
    nb->owned = 1;
    return 1;
}

DPUF_EXPORT DpufToolsModel* dpuf_tools_open_container(const char* path, int32_t verify,
                                                      int32_t max_seq_len, int32_t* status) {
    crc_init();
    *status = 0;
    int fd = open(path, O_RDONLY);
    if (fd < 0) { *status = -1; return NULL; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) { close(fd); *status = -1; return NULL; }
    uint8_t* base = (uint8_t*)mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) { *status = -1; return NULL; }
    DpufToolsModel* m = (DpufToolsModel*)calloc(1, sizeof(DpufToolsModel));
    m->map_base = base;
    m->map_size = (size_t)st.st_size;
    m->tied = 1;
    uint32_t hdr_crc, hlen;
    memcpy(&hdr_crc, base + 12, 4);
    memcpy(&hlen, base + 20, 4);
    if (memcmp(base, "DPUF0001", 8) != 0 && memcmp(base, "LRFLAC03", 8) != 0) { *status = -2; goto fail; }
    if (24u + (uint64_t)hlen > m->map_size) { *status = -3; goto fail; }
    if (crc32_update(0, base + 24, hlen) != hdr_crc) { *status = -4; goto fail; }
    if (!parse_header(m, (const char*)base + 24, hlen, 24u + hlen)) { *status = -5; goto fail; }
    if (max_seq_len > 0) m->cfg.max_seq_len = max_seq_len;
    m->cfg.n_threads = 8;
    if (!bind_all(m, verify)) { *status = -6; goto fail; }
    return m;
fail:
    dpuf_tools_free_model(m);
    return NULL;
}

DPUF_EXPORT void dpuf_tools_free_model(DpufToolsModel* m) {
    if (!m) return;
    for (int32_t i = 0; i < m->n_blobs; i++) {
        if (m->blobs[i].owned) free(m->blobs[i].data);
        free(m->blobs[i].name);
    }
    free(m->blobs);
    for (int32_t i = 0; i < m->n_owned_f; i++) free(m->owned_f[i]);
    free(m->owned_f);
    free(m->layers);
    if (m->map_base) munmap(m->map_base, m->map_size);
    free(m);
}

DPUF_EXPORT const DpufModelConfig* dpuf_tools_model_cfg(const DpufToolsModel* m) { return &m->cfg; }
DPUF_EXPORT const DpufLayerWeights* dpuf_tools_model_layers(const DpufToolsModel* m) { return m->layers; }
DPUF_EXPORT const DpufWeightDesc* dpuf_tools_model_tok(const DpufToolsModel* m) { return &m->tok; }
DPUF_EXPORT const DpufWeightDesc* dpuf_tools_model_lm(const DpufToolsModel* m) { return &m->lm; }
DPUF_EXPORT const float* dpuf_tools_model_out_norm(const DpufToolsModel* m) { return m->out_norm; }
DPUF_EXPORT int32_t dpuf_tools_model_healed(const DpufToolsModel* m) { return m->healed; }

static uint64_t desc_bytes(const DpufWeightDesc* d) { return d->tile_offsets[d->n_tiles]; }

/* Bytes of mode 12 tile payload a single decode step streams: every layer
 * matrix plus the LM head (tiles incl. 16-byte headers and 64-byte padding). */
DPUF_EXPORT uint64_t dpuf_tools_model_weight_bytes(const DpufToolsModel* m) {
    uint64_t s = desc_bytes(&m->lm);
    for (int32_t l = 0; l < m->cfg.num_layers; l++) {
        const DpufLayerWeights* lw = &m->layers[l];
        s += desc_bytes(&lw->w_q) + desc_bytes(&lw->w_k) + desc_bytes(&lw->w_v) + desc_bytes(&lw->w_o) +
             desc_bytes(&lw->w_gate) + desc_bytes(&lw->w_up) + desc_bytes(&lw->w_down);
    }
    return s;
}
