/*
 * dpuf_crc.c -- host-side tile integrity checks of the C ABI.
 *
 * dpuf_crc32_bytes, dpuf_qr_verify_tiles and dpuf_qr_verify_tiles_ex keep the
 * semantics of reference dpuf_avx2.c:347-398 and 846-908: CRC32 (poly
 * 0xEDB88320) of each tile body, compared with the tile header's crc field.
 * They run on the host because they belong to weight ingest (dpuf-cli.c calls
 * them while binding tensors, before dpuf_engine_create), not to the token
 * loop.  Body sizes per mode follow the tile layouts of dpuf_format.py:940-963.
 */
#include <stdlib.h>
#include <string.h>
#include "../../include/dpuf_kernels.h"
#ifdef DPUF_WITH_HIP  /* the build inside libdpuf_amd.so (libdpuf_tools.so has no GPU code) */
#include "../../include/dpuf_amd.h"
#include "hip_layer.h"
#endif

static uint32_t g_tab[256];
static volatile int g_ready = 0;

static void tab_init(void) {
    if (g_ready) return;
    for (uint32_t i = 0; i < 256; i++) {
        uint32_t c = i;
        for (int k = 0; k < 8; k++) c = (c & 1u) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
        g_tab[i] = c;
    }
    g_ready = 1;
}

DPUF_EXPORT uint32_t dpuf_crc32_bytes(const uint8_t* data, uint32_t len) {
    tab_init();
    uint32_t crc = 0xFFFFFFFFu;
    for (uint32_t i = 0; i < len; i++) crc = g_tab[(crc ^ data[i]) & 0xFFu] ^ (crc >> 8);
    return crc ^ 0xFFFFFFFFu;
}

static uint32_t body_bytes(int32_t mode, const DpufQrTileHdr* th, int32_t cols) {
    size_t n_r = th->n_rows;
    size_t n_8g = (n_r + 7) / 8;
    switch (mode) {
    case DPUF_MODE_QR_ZD4:
        return (uint32_t)(n_r * 4u + (n_r * (size_t)cols + 1u) / 2u + th->n_over8 + (size_t)th->n_super16 * 2u);
    case DPUF_MODE_QR_SPLIT4:
        return (uint32_t)(n_r * 6u + (n_r * (size_t)cols) / 2u + (size_t)th->n_over8 * 2u + (size_t)th->n_super16 * 2u);
    case DPUF_MODE_QR_HAD4:
        return (uint32_t)(n_r * (size_t)(cols >> 5) * 2u + (n_r * (size_t)cols) / 2u);
    case DPUF_MODE_QR_Q8:
        return (uint32_t)(n_r * (size_t)(cols >> 5) * 2u + n_r * (size_t)cols);
    case DPUF_MODE_QR_HAD4_PACKED:
        return (uint32_t)(n_8g * (size_t)(cols >> 5) * 144u);
    case DPUF_MODE_QR_HAD4_ASYM:
        return (uint32_t)(n_8g * (size_t)(cols >> 6) * 288u);
    case DPUF_MODE_QR_HAD6:
        return (uint32_t)(n_8g * (size_t)(cols >> 6) * 416u);
    default:
        return 0;
    }
}

DPUF_EXPORT int32_t dpuf_qr_verify_tiles_ex(int32_t mode, int32_t n_tiles, int32_t cols,
                                            const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                            uint8_t* tile_ok_out) {
    tab_init();
    int32_t bad = 0;
    int32_t t;
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 4) if (n_tiles >= 16)
    for (t = 0; t < n_tiles; t++) {
        const uint8_t* tp = tensor_base + tile_offsets[t];
        DpufQrTileHdr th;
        memcpy(&th, tp, sizeof th);
        uint32_t calc = dpuf_crc32_bytes(tp + sizeof(DpufQrTileHdr), body_bytes(mode, &th, cols));
        uint8_t ok = (calc == th.tile_crc32) ? 1u : 0u;
        tile_ok_out[t] = ok;
        if (!ok) bad += 1;
    }
    return bad;
}

DPUF_EXPORT int32_t dpuf_qr_verify_tiles(int32_t n_tiles, int32_t cols, const uint8_t* tensor_base,
                                         const uint64_t* tile_offsets, uint8_t* tile_ok_out) {
    return dpuf_qr_verify_tiles_ex(DPUF_MODE_QR_ZD4, n_tiles, cols, tensor_base, tile_offsets, tile_ok_out);
}

#ifdef DPUF_WITH_HIP
/* The same check on the GPU: the host reads each tile header for its body
 * range and stored CRC, the tile region goes to HBM in one copy and one
 * workgroup per tile computes the CRC (dpuf_hip_crc_tiles). */
static void* g_crc_stream = NULL;

DPUF_EXPORT int32_t dpuf_amd_verify_tiles_device(int32_t mode, int32_t n_tiles, int32_t cols,
                                                 const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                                 uint8_t* tile_ok_out) {
    if (n_tiles <= 0) return 0;
    if (!tensor_base || !tile_offsets || !tile_ok_out || cols <= 0 || dpuf_hip_device_count() <= 0) return -1;
    if (!g_crc_stream) g_crc_stream = dpuf_hip_stream_create();
    void* s = g_crc_stream;
    if (!s) return -1;
    uint64_t* off = (uint64_t*)malloc((size_t)n_tiles * 8);
    uint32_t* len = (uint32_t*)malloc((size_t)n_tiles * 4);
    uint32_t* want = (uint32_t*)malloc((size_t)n_tiles * 4);
    int32_t rc = -1;
    uint8_t *d_base = NULL, *d_ok = NULL;
    uint64_t *d_off = NULL;
    uint32_t *d_len = NULL, *d_want = NULL;
    if (off && len && want) {
        uint64_t end = 0;
        for (int32_t t = 0; t < n_tiles; t++) {
            DpufQrTileHdr th;
            memcpy(&th, tensor_base + tile_offsets[t], sizeof th);
            off[t] = tile_offsets[t] + sizeof(DpufQrTileHdr);
            len[t] = body_bytes(mode, &th, cols);
            want[t] = th.tile_crc32;
            if (off[t] + len[t] > end) end = off[t] + len[t];
        }
        d_base = (uint8_t*)dpuf_hip_malloc((size_t)end);
        d_off = (uint64_t*)dpuf_hip_malloc((size_t)n_tiles * 8);
        d_len = (uint32_t*)dpuf_hip_malloc((size_t)n_tiles * 4);
        d_want = (uint32_t*)dpuf_hip_malloc((size_t)n_tiles * 4);
        d_ok = (uint8_t*)dpuf_hip_malloc((size_t)n_tiles);
        if (d_base && d_off && d_len && d_want && d_ok) {
            dpuf_hip_h2d(d_base, tensor_base, (size_t)end, s);
            dpuf_hip_h2d(d_off, off, (size_t)n_tiles * 8, s);
            dpuf_hip_h2d(d_len, len, (size_t)n_tiles * 4, s);
            dpuf_hip_h2d(d_want, want, (size_t)n_tiles * 4, s);
            dpuf_hip_crc_tiles(s, d_base, d_off, d_len, d_want, d_ok, n_tiles);
            dpuf_hip_d2h(tile_ok_out, d_ok, (size_t)n_tiles, s);
            if (dpuf_hip_sync(s) == 0) {
                rc = 0;
                for (int32_t t = 0; t < n_tiles; t++) rc += tile_ok_out[t] ? 0 : 1;
            }
        }
    }
    dpuf_hip_free(d_base);
    dpuf_hip_free(d_off);
    dpuf_hip_free(d_len);
    dpuf_hip_free(d_want);
    dpuf_hip_free(d_ok);
    free(off);
    free(len);
    free(want);
    return rc;
}
#endif
