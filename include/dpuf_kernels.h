/*
 * dpuf_kernels.h -- C ABI of the MI355X DPUF token loop (Modes 12, 13, 14).
 *
 * This header is the drop-in boundary.  Every type and entry point below keeps
 * the layout, the argument meaning and the return codes of the reference
 * header (dpuf_kernels.h in dulePan/dpuf), so that dpuf-cli.c and the Python
 * ctypes host link against libdpuf_amd.so unchanged.  The bodies are new:
 * weights live in HBM, every compute entry point runs hand-written gfx950 HIP
 * kernels, and nothing here computes on the CPU except the CRC32 tile check,
 * which is host ingest in the reference as well.
 *
 * The Hadamard-4bit packed format (mode 12) and the asymmetric blk64 4-bit
 * and 6-bit formats (modes 13, 14; the had4p-hybrid packing) are
 * implemented, mixed freely per matrix.  Weight descriptors of any other mode
 * make dpuf_engine_create return NULL.
 */
#ifndef DPUF_KERNELS_H
#define DPUF_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#define DPUF_EXPORT __attribute__((visibility("default")))

/* Mode numbers of the QR-tiled container (reference dpuf_kernels.h:29-37). */
enum {
    DPUF_MODE_QR_ZD4         = 8,
    DPUF_MODE_QR_SPLIT4      = 9,
    DPUF_MODE_QR_HAD4        = 10,
    DPUF_MODE_QR_Q8          = 11,
    DPUF_MODE_QR_HAD4_PACKED = 12,
    DPUF_MODE_QR_HAD4_ASYM   = 13,
    DPUF_MODE_QR_HAD6        = 14
};

/* KV cache element type (reference dpuf_kernels.h:39-42). */
enum {
    DPUF_KV_F32 = 0,
    DPUF_KV_Q8  = 1
};

/* 16-byte header in front of every QR tile (reference dpuf_kernels.h:44-51). */
#pragma pack(push, 1)
typedef struct {
    uint32_t tile_crc32;   /* CRC32 of the tile body that follows            */
    uint16_t n_rows;       /* rows stored in this tile (<= 16)                */
    uint16_t flags;        /* 0                                               */
    uint32_t n_over8;      /* 0 for modes 12-14                               */
    uint32_t n_super16;    /* 0 for modes 12-14                               */
} DpufQrTileHdr;
#pragma pack(pop)

/* Borrowed view of one QR-tiled weight matrix (reference dpuf_kernels.h:53-62).
 * 48 bytes on LP64.  For modes 12-14 col_scale is NULL and sign_bits holds
 * cols/8 bytes (bit c%8 of byte c/8 set = negate column c). */
typedef struct {
    int32_t mode;
    int32_t rows;
    int32_t cols;
    int32_t n_tiles;
    const uint8_t*  tensor_base;   /* tile t starts at tensor_base + tile_offsets[t] */
    const uint64_t* tile_offsets;  /* n_tiles + 1 entries                            */
    const float*    col_scale;
    const uint8_t*  sign_bits;
} DpufWeightDesc;

/* Model shape and options (reference dpuf_kernels.h:64-87), 92 bytes. */
typedef struct {
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t num_layers;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t vocab_size;
    int32_t max_seq_len;
    int32_t has_qk_norm;
    float   rms_eps;
    float   rope_theta;
    int32_t n_threads;          /* kept for layout; the GPU engine ignores it   */
    int32_t use_llama3_rope;
    float   rope_factor;
    float   rope_low_freq;
    float   rope_high_freq;
    int32_t rope_orig_max_pos;
    int32_t kv_type;            /* DPUF_KV_F32 or DPUF_KV_Q8 (int8 per 32 values) */
    int32_t has_mrope;          /* must be 0 (multimodal RoPE is not built)      */
    int32_t mrope_section[3];
    int32_t mrope_interleaved;
} DpufModelConfig;

/* Per-layer weights (reference dpuf_kernels.h:89-101), 368 bytes on LP64. */
typedef struct {
    const float* attn_norm;
    const float* attn_q_norm;
    const float* attn_k_norm;
    const float* ffn_norm;
    DpufWeightDesc w_q;
    DpufWeightDesc w_k;
    DpufWeightDesc w_v;
    DpufWeightDesc w_o;
    DpufWeightDesc w_gate;
    DpufWeightDesc w_up;
    DpufWeightDesc w_down;
} DpufLayerWeights;

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Host ingest helpers (reference dpuf_avx2.c:347-398, 846-908) -------- */

/* Standard CRC32 (poly 0xEDB88320, init/xorout 0xFFFFFFFF).
 * Replaces reference dpuf_kernels.h:105. */
DPUF_EXPORT uint32_t dpuf_crc32_bytes(const uint8_t* data, uint32_t len);

/* Verifies mode-8 tile bodies; kept for the ABI (reference dpuf_kernels.h:107-113). */
DPUF_EXPORT int32_t dpuf_qr_verify_tiles(int32_t n_tiles, int32_t cols,
                                         const uint8_t* tensor_base,
                                         const uint64_t* tile_offsets,
                                         uint8_t* tile_ok_out);

/* Checks every tile's CRC32; tile_ok_out[t] = 1 when intact.  Returns the
 * number of bad tiles.  Replaces reference dpuf_kernels.h:115-122; called by
 * dpuf-cli.c:1671,1720 while binding weights. */
DPUF_EXPORT int32_t dpuf_qr_verify_tiles_ex(int32_t mode, int32_t n_tiles, int32_t cols,
                                            const uint8_t* tensor_base,
                                            const uint64_t* tile_offsets,
                                            uint8_t* tile_ok_out);

/* ---- Mode 12 compute entry points (host pointers; run on the GPU) -------- */

/* x_out = FWHT64(sign (.) x_in), per 64-column block, scaled by 1/8.
 * Replaces reference dpuf_kernels.h:134-139 (dpuf_avx2.c:774-788). */
DPUF_EXPORT void dpuf_fwht64_sign_f32(int32_t cols, const float* x_in,
                                      const uint8_t* sign_bits, float* x_out);

/* Activation prep: FWHT64 + sign, then per-32 int8 quantisation.
 * pack_slab = 0: x_out int8[cols], x_scale_out f32[cols/32], x_sum8_out i32[cols/32] (mc = 1).
 * pack_slab = 1: slab of mc <= 6 rows, x_out as [n_blk][8 words][6] int32,
 *                scales and sums as [n_blk][6].
 * Replaces reference dpuf_kernels.h:242-252 (dpuf_avx2.c:2364-2449). */
DPUF_EXPORT void dpuf_prep_had4_packed_slab(int32_t mc, int32_t cols,
                                            const float* x_slab_f32,
                                            const uint8_t* sign_bits,
                                            float* f_scratch,
                                            int8_t* x_out,
                                            float* x_scale_out,
                                            int32_t* x_sum8_out,
                                            int32_t pack_slab);

/* out rows of tiles [t_start, t_end) from prepped activations (row layout for
 * M == 1, slab layout for M > 1).  out is [M][rows] (M > 1) or [rows].
 * Replaces reference dpuf_kernels.h:254-266 (dpuf_avx2.c:2585-2676). */
DPUF_EXPORT void dpuf_matmul_qr_hadamard4_packed_tile_range(
    int32_t M, int32_t rows, int32_t cols, int32_t t_start, int32_t t_end,
    const int8_t* x_q8, const float* x_blk_scale, const int32_t* x_sum8,
    const uint8_t* tensor_base, const uint64_t* tile_offsets, float* out);

/* out[M][rows] = W x for fp32 x[M][cols]: prep + matmul in one call.
 * Entry of the isolated-GEMV workload.  Replaces reference
 * dpuf_kernels.h:267-271 (dpuf_avx2.c:2678-2736). */
DPUF_EXPORT void dpuf_matmul_qr_hadamard4_packed_f32(
    int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
    const float* x_in, const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* Embedding rows: sign (.) FWHT64((u - 8) * scale).
 * Replaces reference dpuf_kernels.h:273-277 (dpuf_avx2.c:2738-2783). */
DPUF_EXPORT void dpuf_embed_qr_hadamard4_packed_f32(
    int32_t n_tokens, int32_t cols, const int32_t* token_ids,
    const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* ---- Modes 13 / 14: asymmetric blk64 4-bit / 6-bit ----------------------
 * Tile groups of 8 rows: [cols/64][16] fp16 (d of rows 0..7, then m), the
 * 4-bit codes in the mode 12 nibble interleave, and for mode 14 the 2-bit
 * high planes.  Row value (rotated) = m + u * d per 64-column block.  The
 * activations are prepped as for mode 12 (dpuf_prep_had4_packed_slab). */

/* Replaces reference dpuf_kernels.h:280-284 (dpuf_avx2.c:2947-3074). */
DPUF_EXPORT void dpuf_matmul_qr_had4_asym_tile_range(
    int32_t M, int32_t rows, int32_t cols, int32_t t_start, int32_t t_end,
    const int8_t* x_q8, const float* x_blk_scale, const int32_t* x_sum8,
    const uint8_t* tensor_base, const uint64_t* tile_offsets, float* out);

/* Replaces reference dpuf_kernels.h:286-290 (dpuf_avx2.c:3084-3136). */
DPUF_EXPORT void dpuf_matmul_qr_had4_asym_f32(
    int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
    const float* x_in, const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* Replaces reference dpuf_kernels.h:292-296 (dpuf_avx2.c:3146-3213). */
DPUF_EXPORT void dpuf_embed_qr_had4_asym_f32(
    int32_t n_tokens, int32_t cols, const int32_t* token_ids,
    const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* Replaces reference dpuf_kernels.h:298-302 (dpuf_avx2.c:2947-3082). */
DPUF_EXPORT void dpuf_matmul_qr_had6_tile_range(
    int32_t M, int32_t rows, int32_t cols, int32_t t_start, int32_t t_end,
    const int8_t* x_q8, const float* x_blk_scale, const int32_t* x_sum8,
    const uint8_t* tensor_base, const uint64_t* tile_offsets, float* out);

/* Replaces reference dpuf_kernels.h:304-308 (dpuf_avx2.c:3084-3144). */
DPUF_EXPORT void dpuf_matmul_qr_had6_f32(
    int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
    const float* x_in, const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* Replaces reference dpuf_kernels.h:310-314 (dpuf_avx2.c:3146-3221). */
DPUF_EXPORT void dpuf_embed_qr_had6_f32(
    int32_t n_tokens, int32_t cols, const int32_t* token_ids,
    const uint8_t* tensor_base, const uint64_t* tile_offsets,
    const uint8_t* sign_bits, float* out);

/* Mode dispatcher for embeddings (modes 12, 13, 14 here; other modes write
 * nothing).  Replaces reference dpuf_kernels.h:170-176 (dpuf_avx2.c:2044-2067). */
DPUF_EXPORT void dpuf_embed_qr_any_f32(const DpufWeightDesc* w, int32_t n_tokens,
                                       const int32_t* token_ids, float* out,
                                       float* scratch_f32);

/* ---- Persistent engine (reference dpuf_kernels.h:316-360) ---------------- */

/* Copies *cfg and layers[0..num_layers); everything the descriptors point to
 * is read once and uploaded to HBM.  Returns NULL on bad arguments, a mode
 * other than 12, 13, 14, or allocation failure.  Reads DPUF_SWIGLU_DEADZONE
 * here. */
DPUF_EXPORT void* dpuf_engine_create(const DpufModelConfig* cfg,
                                     const DpufLayerWeights* layers,
                                     const DpufWeightDesc* w_tok_embd,
                                     const DpufWeightDesc* w_lm_head,
                                     const float* output_norm);
DPUF_EXPORT void    dpuf_engine_destroy(void* handle);
DPUF_EXPORT void    dpuf_engine_reset_cache(void* handle);
DPUF_EXPORT int32_t dpuf_engine_set_slot(void* handle, int32_t slot_id);
DPUF_EXPORT int32_t dpuf_engine_get_slot(void* handle);
DPUF_EXPORT void    dpuf_engine_reset_slot(void* handle, int32_t slot_id);
DPUF_EXPORT size_t  dpuf_engine_slot_memory(void* handle);
DPUF_EXPORT int32_t dpuf_engine_num_slots(void* handle);
DPUF_EXPORT int32_t dpuf_engine_freeze_prefix(void* handle, int32_t prefix_id, int32_t prefix_len);
DPUF_EXPORT int32_t dpuf_engine_apply_prefix(void* handle, int32_t slot_id, int32_t prefix_id);
DPUF_EXPORT int32_t dpuf_engine_get_prefix_len(void* handle, int32_t prefix_id);

/* Return codes: 0 ok; -1 null handle/ids/logits; -2 n_tokens not in
 * [1, DPUF_AMD_MAX_BATCH]; -3 pos0 < 0 or pos0 + n_tokens > max_seq_len;
 * -4 a token id outside [0, vocab_size) (the reference reads out of bounds
 * there); -5 M-RoPE / DeepStack inputs (not built); -6 device error.
 * only_last_logits: 0 = logits for every row ([n][V]), 1 = last row ([V]),
 * 2 = no LM head (KV-only chunk; logits_out may be NULL).
 * Reads DPUF_PREFILL_KEEP_TILES / DPUF_GEN_KEEP_TILES / DPUF_EARLY_TILES /
 * DPUF_EARLY_MARGIN on every call. */
DPUF_EXPORT int32_t dpuf_engine_forward_batch(void* handle, int32_t n_tokens,
                                              const int32_t* token_ids, int32_t pos0,
                                              int32_t only_last_logits, float* logits_out);
DPUF_EXPORT int32_t dpuf_engine_forward_batch_ex(void* handle, int32_t n_tokens,
                                                 const int32_t* token_ids, int32_t pos0,
                                                 const float* embeds_in,
                                                 const int32_t* pos_t,
                                                 const int32_t* pos_h,
                                                 const int32_t* pos_w,
                                                 const float* const* deepstack_in,
                                                 int32_t only_last_logits,
                                                 float* logits_out);
DPUF_EXPORT int32_t dpuf_engine_forward_token(void* handle, int32_t token_id,
                                              int32_t pos, float* logits_out);

#ifdef __cplusplus
}
#endif

#endif /* DPUF_KERNELS_H */
