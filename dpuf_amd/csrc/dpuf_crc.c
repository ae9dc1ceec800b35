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
#include <string.h>
#include "../../include/dpuf_kernels.h"

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
