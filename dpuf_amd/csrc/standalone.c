/*
 * standalone.c -- the mode 12, 13 and 14 entry points of the ABI that take
 * host pointers (reference dpuf_avx2.c:774-788, 2364-2449, 2585-2783,
 * 2947-3221).  Each call
 * validates its tiles on the host, stages inputs to HBM, runs the same HIP
 * kernels as the engine, and copies results back before returning.  They are
 * synchronous and allocate per call; throughput users keep weights resident
 * in an engine instead.
 */
#include <stdlib.h>
#include <string.h>

#include "../../include/dpuf_kernels.h"
#include "hip_layer.h"

static void* g_stream = NULL;

/* The library's stream for the host-pointer entries; also starts the call's
 * error state afresh. */
static void* stream(void) {
    dpuf_hip_clear_error();
    if (!g_stream && dpuf_hip_device_count() > 0) g_stream = dpuf_hip_stream_create();
    return g_stream;
}

/* A call that validated its arguments but could not finish (allocation,
 * runtime or kernel failure) writes NaN to every output it owns, so the
 * failure cannot pass for a result; dpuf_amd_last_error() says why. */
static void fail_rows(float* out, int32_t M, int32_t ld, int32_t r0, int32_t r1) {
    const uint32_t nan_bits = 0x7FC00000u;
    float nanv;
    memcpy(&nanv, &nan_bits, 4);
    for (int32_t m = 0; m < M; m++)
        for (int32_t r = r0; r < r1; r++) out[(size_t)m * ld + r] = nanv;
}

/* Largest token count of one GEMM launch at K columns (M * K < 2^30). */
static int32_t max_chunk(int32_t M, int32_t cols) {
    const int64_t cap = ((int64_t)1 << 30) / cols - 1;
    return (int64_t)M < cap ? M : (int32_t)cap;
}

/* Checks tiles [t0, t1) of a mode 12 / 13 / 14 payload (tile t holds
 * min(16, rows - 16t) rows, its groups lie inside the byte range) and
 * returns the byte range [*lo, *hi). */
static int check_tiles(int32_t mode, int32_t rows, int32_t cols, int32_t t0, int32_t t1, const uint8_t* base,
                       const uint64_t* offs, uint64_t* lo, uint64_t* hi) {
    if (cols <= 0 || (cols % 64) != 0 || t0 < 0 || t1 <= t0 || !base || !offs) return 0;
    const uint64_t grp = (uint64_t)(cols / 32) * (uint64_t)dpuf_grp_unit(mode);
    *lo = offs[t0];
    *hi = offs[t1];
    if (*hi < *lo) return 0;
    for (int32_t t = t0; t < t1; t++) {
        if (offs[t] < *lo || offs[t] + 16 > *hi || ((offs[t] - *lo) % 16) != 0) return 0;
        DpufQrTileHdr th;
        memcpy(&th, base + offs[t], sizeof th);
        const int64_t want = (int64_t)rows - (int64_t)t * 16 < 16 ? (int64_t)rows - (int64_t)t * 16 : 16;
        if (want < 1 || th.n_rows != want) return 0;
        if (offs[t] + 16 + (uint64_t)((th.n_rows + 7) / 8) * grp > *hi) return 0;
    }
    return 1;
}

typedef struct {
    void* groups;
    void* sign;
    DpufDevW w;   /* row 0 of w is row 16 * t0 of the matrix */
} Staged;

/* Uploads tiles [t0, t1) and converts them to the row-block layout. */
static int stage_weights(int32_t mode, int32_t rows, int32_t cols, int32_t t0, int32_t t1, const uint8_t* base,
                         const uint64_t* offs, const uint8_t* sign, Staged* st) {
    uint64_t lo, hi;
    memset(st, 0, sizeof *st);
    if (!check_tiles(mode, rows, cols, t0, t1, base, offs, &lo, &hi)) return 0;
    void* s = stream();
    const int32_t nt = t1 - t0, n_blk = cols / 32;
    const int32_t rows_st = (rows < 16 * t1 ? rows : 16 * t1) - 16 * t0;
    const int32_t n_groups = (rows_st + 7) / 8;
    uint64_t* rel = (uint64_t*)calloc((size_t)nt + 1, 8);
    if (!rel) return 0;
    for (int32_t t = 0; t <= nt; t++) rel[t] = offs[t0 + t] - lo;
    void* d_raw = dpuf_hip_malloc((size_t)(hi - lo));
    void* d_offs = dpuf_hip_malloc(((size_t)nt + 1) * 8);
    st->groups = dpuf_hip_malloc((size_t)n_groups * n_blk * dpuf_grp_unit(mode));
    if (sign) st->sign = dpuf_hip_malloc((size_t)cols / 8);
    int ok = d_raw && d_offs && st->groups && (!sign || st->sign);
    if (ok) {
        dpuf_hip_h2d(d_raw, base + lo, (size_t)(hi - lo), s);
        dpuf_hip_h2d(d_offs, rel, ((size_t)nt + 1) * 8, s);
        if (sign) dpuf_hip_h2d(st->sign, sign, (size_t)cols / 8, s);
        dpuf_hip_relayout(s, (const uint8_t*)d_raw, (const uint64_t*)d_offs, n_groups, n_blk, mode,
                          (uint8_t*)st->groups);
        ok = dpuf_hip_sync(s) == 0;
    }
    free(rel);
    dpuf_hip_free(d_raw);
    dpuf_hip_free(d_offs);
    if (!ok) {
        dpuf_hip_free(st->groups);
        dpuf_hip_free(st->sign);
        memset(st, 0, sizeof *st);
        return 0;
    }
    st->w.g = (const uint8_t*)st->groups;
    st->w.sign = (const uint8_t*)st->sign;
    st->w.rows = rows_st;
    st->w.cols = cols;
    st->w.n_groups = n_groups;
    st->w.mode = mode;
    return 1;
}

static void unstage(Staged* st) {
    dpuf_hip_free(st->groups);
    dpuf_hip_free(st->sign);
}

/* M > 1 also gets the fp16 copy of q that the slab GEMM reads. */
static int prep_alloc(DpufPrep* p, int32_t M, int32_t K) {
    p->q = (int8_t*)dpuf_hip_malloc((size_t)M * K);
    p->s = (float*)dpuf_hip_malloc((size_t)M * (K / 32) * 4);
    p->m = (int32_t*)dpuf_hip_malloc((size_t)M * (K / 32) * 4);
    p->h = M > 1 ? (uint16_t*)dpuf_hip_malloc((size_t)M * K * 2) : NULL;
    return p->q && p->s && p->m && (M == 1 || p->h);
}

static void prep_free(DpufPrep* p) {
    dpuf_hip_free(p->q);
    dpuf_hip_free(p->s);
    dpuf_hip_free(p->m);
    dpuf_hip_free(p->h);
}

DPUF_EXPORT void dpuf_fwht64_sign_f32(int32_t cols, const float* x_in, const uint8_t* sign_bits, float* x_out) {
    void* s = stream();
    if (!s || cols <= 0 || (cols % 64) != 0 || !x_in || !x_out) return;
    float* dx = (float*)dpuf_hip_malloc((size_t)cols * 4);
    float* dy = (float*)dpuf_hip_malloc((size_t)cols * 4);
    void* ds = sign_bits ? dpuf_hip_malloc((size_t)cols / 8) : NULL;
    if (dx && dy && (!sign_bits || ds)) {
        dpuf_hip_h2d(dx, x_in, (size_t)cols * 4, s);
        if (ds) dpuf_hip_h2d(ds, sign_bits, (size_t)cols / 8, s);
        dpuf_hip_fwht_sign(s, 1, cols, dx, (const uint8_t*)ds, dy);
        dpuf_hip_d2h(x_out, dy, (size_t)cols * 4, s);
        dpuf_hip_sync(s);
    }
    dpuf_hip_free(dx); dpuf_hip_free(dy); dpuf_hip_free(ds);
}

DPUF_EXPORT void dpuf_prep_had4_packed_slab(int32_t mc, int32_t cols, const float* x_slab_f32,
                                            const uint8_t* sign_bits, float* f_scratch, int8_t* x_out,
                                            float* x_scale_out, int32_t* x_sum8_out, int32_t pack_slab) {
    void* s = stream();
    if (!s || mc <= 0 || mc > 6 || cols <= 0 || (cols % 64) != 0 || !x_slab_f32 || !x_out || !x_scale_out ||
        !x_sum8_out)
        return;
    const int32_t nb = cols / 32;
    float* dx = (float*)dpuf_hip_malloc((size_t)mc * cols * 4);
    float* df = (float*)dpuf_hip_malloc((size_t)mc * cols * 4);
    void* ds = sign_bits ? dpuf_hip_malloc((size_t)cols / 8) : NULL;
    DpufPrep rows = {0, 0, 0, 0};
    int32_t* sq = (int32_t*)dpuf_hip_malloc((size_t)nb * 192);
    float* ss = (float*)dpuf_hip_malloc((size_t)nb * 6 * 4);
    int32_t* sm = (int32_t*)dpuf_hip_malloc((size_t)nb * 6 * 4);
    if (dx && df && (!sign_bits || ds) && prep_alloc(&rows, mc, cols) && sq && ss && sm) {
        dpuf_hip_h2d(dx, x_slab_f32, (size_t)mc * cols * 4, s);
        if (ds) dpuf_hip_h2d(ds, sign_bits, (size_t)cols / 8, s);
        dpuf_hip_prep(s, mc, cols, dx, (const uint8_t*)ds, rows);
        if (f_scratch) {
            dpuf_hip_fwht_sign(s, mc, cols, dx, (const uint8_t*)ds, df);
            dpuf_hip_d2h(f_scratch, df, (size_t)mc * cols * 4, s);
        }
        if (pack_slab) {
            /* token lanes j >= mc keep the caller's previous contents */
            dpuf_hip_h2d(sq, x_out, (size_t)nb * 192, s);
            dpuf_hip_h2d(ss, x_scale_out, (size_t)nb * 6 * 4, s);
            dpuf_hip_h2d(sm, x_sum8_out, (size_t)nb * 6 * 4, s);
            dpuf_hip_slab_pack(s, mc, cols, rows, sq, ss, sm);
            dpuf_hip_d2h(x_out, sq, (size_t)nb * 192, s);
            dpuf_hip_d2h(x_scale_out, ss, (size_t)nb * 6 * 4, s);
            dpuf_hip_d2h(x_sum8_out, sm, (size_t)nb * 6 * 4, s);
        } else {
            /* row layout: every row writes the same outputs, the last one stays */
            const size_t r = (size_t)(mc - 1);
            dpuf_hip_d2h(x_out, rows.q + r * cols, (size_t)cols, s);
            dpuf_hip_d2h(x_scale_out, rows.s + r * nb, (size_t)nb * 4, s);
            dpuf_hip_d2h(x_sum8_out, rows.m + r * nb, (size_t)nb * 4, s);
        }
        dpuf_hip_sync(s);
    }
    dpuf_hip_free(dx); dpuf_hip_free(df); dpuf_hip_free(ds);
    dpuf_hip_free(sq); dpuf_hip_free(ss); dpuf_hip_free(sm);
    prep_free(&rows);
}

/* Copies rows [r0, r1) of M output rows of width `rows` back to the host. */
static void fetch_rows(float* out, const float* dout, int32_t M, int32_t rows, int32_t r0, int32_t r1, void* s) {
    if (r1 <= r0) return;
    if (r0 == 0 && r1 == rows) {
        dpuf_hip_d2h(out, dout, (size_t)M * rows * 4, s);
        return;
    }
    for (int32_t m = 0; m < M; m++)
        dpuf_hip_d2h(out + (size_t)m * rows + r0, dout + (size_t)m * rows + r0, (size_t)(r1 - r0) * 4, s);
}

/* Tiles [t_start, t_end) of a mode 12 / 13 / 14 matrix from prepped
 * activations (row layout for M == 1, slab layout for M > 1). */
static void tile_range(int32_t mode, int32_t M, int32_t rows, int32_t cols, int32_t t_start, int32_t t_end,
                       const int8_t* x_q8, const float* x_blk_scale, const int32_t* x_sum8,
                       const uint8_t* tensor_base, const uint64_t* tile_offsets, float* out) {
    void* s = stream();
    if (!s || M <= 0 || rows <= 0 || t_start < 0 || t_end <= t_start || (int64_t)t_start * 16 >= rows || !x_q8 ||
        !x_blk_scale || !x_sum8 || !out)
        return;
    if ((int64_t)t_end * 16 > (int64_t)rows + 15) return;
    if ((int64_t)M * cols >= ((int64_t)1 << 30)) return; /* the slab inputs are one block */
    const int32_t r1 = t_end * 16 < rows ? t_end * 16 : rows;
    Staged st;
    if (!stage_weights(mode, rows, cols, t_start, t_end, tensor_base, tile_offsets, NULL, &st)) {
        fail_rows(out, M, rows, t_start * 16, r1);
        return;
    }
    const int32_t nb = cols / 32;
    DpufPrep p = {0, 0, 0, 0};
    float* dout = (float*)dpuf_hip_malloc((size_t)M * rows * 4);
    int32_t* derr = (int32_t*)dpuf_hip_malloc(4);
    int32_t herr = 1;
    if (prep_alloc(&p, M, cols) && dout && derr) {
        dpuf_hip_fill_zero(derr, 4, s);
        dpuf_hip_bind_error_word(derr);
        if (M == 1) {
            dpuf_hip_h2d(p.q, x_q8, (size_t)cols, s);
            dpuf_hip_h2d(p.s, x_blk_scale, (size_t)nb * 4, s);
            dpuf_hip_h2d(p.m, x_sum8, (size_t)nb * 4, s);
        } else {
            const int32_t ns = (M + 5) / 6;
            int32_t* sq = (int32_t*)dpuf_hip_malloc((size_t)ns * nb * 192);
            float* ss = (float*)dpuf_hip_malloc((size_t)ns * nb * 6 * 4);
            int32_t* sm = (int32_t*)dpuf_hip_malloc((size_t)ns * nb * 6 * 4);
            if (sq && ss && sm) {
                dpuf_hip_h2d(sq, x_q8, (size_t)ns * nb * 192, s);
                dpuf_hip_h2d(ss, x_blk_scale, (size_t)ns * nb * 6 * 4, s);
                dpuf_hip_h2d(sm, x_sum8, (size_t)ns * nb * 6 * 4, s);
                dpuf_hip_slab_unpack(s, M, cols, sq, ss, sm, p);
                dpuf_hip_sync(s);
            }
            dpuf_hip_free(sq); dpuf_hip_free(ss); dpuf_hip_free(sm);
        }
        DpufGemvJob j;
        j.w = st.w;
        j.g0 = 0;
        j.g1 = st.w.n_groups;
        j.p = p;
        j.out = dout + (size_t)t_start * 16;
        j.ldo = rows;
        dpuf_hip_gemv(s, M, 1, &j, NULL, 0.0f);
        fetch_rows(out, dout, M, rows, t_start * 16, r1, s);
        dpuf_hip_d2h(&herr, derr, 4, s);
        if (dpuf_hip_sync(s) != 0) herr = 1;
    }
    if (herr != 0) fail_rows(out, M, rows, t_start * 16, r1);
    dpuf_hip_bind_error_word(NULL);
    prep_free(&p);
    dpuf_hip_free(dout);
    dpuf_hip_free(derr);
    unstage(&st);
}

DPUF_EXPORT void dpuf_matmul_qr_hadamard4_packed_tile_range(int32_t M, int32_t rows, int32_t cols, int32_t t_start,
                                                            int32_t t_end, const int8_t* x_q8,
                                                            const float* x_blk_scale, const int32_t* x_sum8,
                                                            const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                                            float* out) {
    tile_range(DPUF_MODE_QR_HAD4_PACKED, M, rows, cols, t_start, t_end, x_q8, x_blk_scale, x_sum8, tensor_base,
               tile_offsets, out);
}

DPUF_EXPORT void dpuf_matmul_qr_had4_asym_tile_range(int32_t M, int32_t rows, int32_t cols, int32_t t_start,
                                                     int32_t t_end, const int8_t* x_q8, const float* x_blk_scale,
                                                     const int32_t* x_sum8, const uint8_t* tensor_base,
                                                     const uint64_t* tile_offsets, float* out) {
    tile_range(DPUF_MODE_QR_HAD4_ASYM, M, rows, cols, t_start, t_end, x_q8, x_blk_scale, x_sum8, tensor_base,
               tile_offsets, out);
}

DPUF_EXPORT void dpuf_matmul_qr_had6_tile_range(int32_t M, int32_t rows, int32_t cols, int32_t t_start,
                                                int32_t t_end, const int8_t* x_q8, const float* x_blk_scale,
                                                const int32_t* x_sum8, const uint8_t* tensor_base,
                                                const uint64_t* tile_offsets, float* out) {
    tile_range(DPUF_MODE_QR_HAD6, M, rows, cols, t_start, t_end, x_q8, x_blk_scale, x_sum8, tensor_base,
               tile_offsets, out);
}

/* out[M][rows] = W x for a mode 12 / 13 / 14 matrix: prep + GEMV / GEMM. */
static void matmul_f32(int32_t mode, int32_t M, int32_t rows, int32_t cols, int32_t n_tiles, const float* x_in,
                       const uint8_t* tensor_base, const uint64_t* tile_offsets, const uint8_t* sign_bits,
                       float* out) {
    void* s = stream();
    if (!s || M <= 0 || rows <= 0 || n_tiles <= 0 || !x_in || !out) return;
    if ((int64_t)n_tiles * 16 > (int64_t)rows + 15 || (int64_t)n_tiles * 16 < rows) return;
    Staged st;
    if (!stage_weights(mode, rows, cols, 0, n_tiles, tensor_base, tile_offsets, sign_bits, &st)) {
        fail_rows(out, M, rows, 0, rows);
        return;
    }
    /* token chunks keep every launch below 2^30 activation bytes; each
     * (row, token) result does not depend on the other tokens */
    const int32_t mc = max_chunk(M, cols);
    DpufPrep p = {0, 0, 0, 0};
    float* dx = (float*)dpuf_hip_malloc((size_t)mc * cols * 4);
    float* dout = (float*)dpuf_hip_malloc((size_t)mc * rows * 4);
    int32_t* derr = (int32_t*)dpuf_hip_malloc(4);
    int32_t herr = 1;
    if (prep_alloc(&p, mc, cols) && dx && dout && derr) {
        dpuf_hip_fill_zero(derr, 4, s);
        dpuf_hip_bind_error_word(derr);
        for (int32_t m0 = 0; m0 < M; m0 += mc) {
            const int32_t n = M - m0 < mc ? M - m0 : mc;
            dpuf_hip_h2d(dx, x_in + (size_t)m0 * cols, (size_t)n * cols * 4, s);
            dpuf_hip_prep(s, n, cols, dx, st.w.sign, p);
            DpufGemvJob j;
            j.w = st.w;
            j.g0 = 0;
            j.g1 = st.w.n_groups;
            j.p = p;
            j.out = dout;
            j.ldo = rows;
            dpuf_hip_gemv(s, n, 1, &j, NULL, 0.0f);
            dpuf_hip_d2h(out + (size_t)m0 * rows, dout, (size_t)n * rows * 4, s);
        }
        dpuf_hip_d2h(&herr, derr, 4, s);
        if (dpuf_hip_sync(s) != 0) herr = 1;
    }
    if (herr != 0) fail_rows(out, M, rows, 0, rows);
    dpuf_hip_bind_error_word(NULL);
    prep_free(&p);
    dpuf_hip_free(dx);
    dpuf_hip_free(dout);
    dpuf_hip_free(derr);
    unstage(&st);
}

DPUF_EXPORT void dpuf_matmul_qr_hadamard4_packed_f32(int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                                                     const float* x_in, const uint8_t* tensor_base,
                                                     const uint64_t* tile_offsets, const uint8_t* sign_bits,
                                                     float* out) {
    matmul_f32(DPUF_MODE_QR_HAD4_PACKED, M, rows, cols, n_tiles, x_in, tensor_base, tile_offsets, sign_bits, out);
}

DPUF_EXPORT void dpuf_matmul_qr_had4_asym_f32(int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                                              const float* x_in, const uint8_t* tensor_base,
                                              const uint64_t* tile_offsets, const uint8_t* sign_bits, float* out) {
    matmul_f32(DPUF_MODE_QR_HAD4_ASYM, M, rows, cols, n_tiles, x_in, tensor_base, tile_offsets, sign_bits, out);
}

DPUF_EXPORT void dpuf_matmul_qr_had6_f32(int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                                         const float* x_in, const uint8_t* tensor_base,
                                         const uint64_t* tile_offsets, const uint8_t* sign_bits, float* out) {
    matmul_f32(DPUF_MODE_QR_HAD6, M, rows, cols, n_tiles, x_in, tensor_base, tile_offsets, sign_bits, out);
}

/* Embedding rows of a mode 12 / 13 / 14 matrix. */
static void embed_f32(int32_t mode, int32_t n_tokens, int32_t cols, const int32_t* token_ids,
                      const uint8_t* tensor_base, const uint64_t* tile_offsets, const uint8_t* sign_bits,
                      float* out) {
    void* s = stream();
    if (!s || n_tokens <= 0 || !token_ids || !out) return;
    int32_t max_id = 0;
    for (int32_t i = 0; i < n_tokens; i++) {
        if (token_ids[i] < 0) return;
        if (token_ids[i] > max_id) max_id = token_ids[i];
    }
    const int32_t nt = max_id / 16 + 1;
    for (int32_t i = 0; i < n_tokens; i++) {
        DpufQrTileHdr th;
        memcpy(&th, tensor_base + tile_offsets[token_ids[i] / 16], sizeof th);
        if (token_ids[i] % 16 >= th.n_rows) return;
    }
    /* rows covered by tiles [0, nt): the last one may be a short final tile */
    DpufQrTileHdr last;
    memcpy(&last, tensor_base + tile_offsets[nt - 1], sizeof last);
    Staged st;
    if (!stage_weights(mode, (nt - 1) * 16 + last.n_rows, cols, 0, nt, tensor_base, tile_offsets, sign_bits, &st))
        return;
    int32_t* dids = (int32_t*)dpuf_hip_malloc((size_t)n_tokens * 4);
    float* dout = (float*)dpuf_hip_malloc((size_t)n_tokens * cols * 4);
    if (dids && dout) {
        dpuf_hip_h2d(dids, token_ids, (size_t)n_tokens * 4, s);
        dpuf_hip_embed(s, st.w, dids, n_tokens, NULL, 0, dout, NULL, NULL, NULL);
        dpuf_hip_d2h(out, dout, (size_t)n_tokens * cols * 4, s);
        dpuf_hip_sync(s);
    }
    dpuf_hip_free(dids);
    dpuf_hip_free(dout);
    unstage(&st);
}

DPUF_EXPORT void dpuf_embed_qr_hadamard4_packed_f32(int32_t n_tokens, int32_t cols, const int32_t* token_ids,
                                                    const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                                    const uint8_t* sign_bits, float* out) {
    embed_f32(DPUF_MODE_QR_HAD4_PACKED, n_tokens, cols, token_ids, tensor_base, tile_offsets, sign_bits, out);
}

DPUF_EXPORT void dpuf_embed_qr_had4_asym_f32(int32_t n_tokens, int32_t cols, const int32_t* token_ids,
                                             const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                             const uint8_t* sign_bits, float* out) {
    embed_f32(DPUF_MODE_QR_HAD4_ASYM, n_tokens, cols, token_ids, tensor_base, tile_offsets, sign_bits, out);
}

DPUF_EXPORT void dpuf_embed_qr_had6_f32(int32_t n_tokens, int32_t cols, const int32_t* token_ids,
                                        const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                        const uint8_t* sign_bits, float* out) {
    embed_f32(DPUF_MODE_QR_HAD6, n_tokens, cols, token_ids, tensor_base, tile_offsets, sign_bits, out);
}

DPUF_EXPORT void dpuf_embed_qr_any_f32(const DpufWeightDesc* w, int32_t n_tokens, const int32_t* token_ids,
                                       float* out, float* scratch_f32) {
    (void)scratch_f32;
    if (!w || (w->mode != DPUF_MODE_QR_HAD4_PACKED && w->mode != DPUF_MODE_QR_HAD4_ASYM &&
               w->mode != DPUF_MODE_QR_HAD6))
        return; /* other modes are not built */
    embed_f32(w->mode, n_tokens, w->cols, token_ids, w->tensor_base, w->tile_offsets, w->sign_bits, out);
}
