/*
 * oracle.h -- CPU restatement of the reference DPUF token loop (modes 12, 13, 14).
 * TEST INFRASTRUCTURE ONLY: used by tests/, the smoke check and the CPU
 * baseline of bench.py as the checker; never linked into libdpuf_amd.so.
 */
#ifndef DPUF_ORACLE_H
#define DPUF_ORACLE_H

#include <stdint.h>
#include "../include/dpuf_kernels.h"

#define ORC_MAX_SLOTS 8
#define ORC_MAX_PREFIXES 8
#define ORC_MAX_BATCH 512

#ifdef __cplusplus
extern "C" {
#endif

typedef struct OrcEngine OrcEngine;

float orc_h2f(uint16_t h);
float orc_exp_poly(float x);
void orc_fwht64(float* y);
void orc_fwht64_sign(int32_t cols, const float* x, const uint8_t* sb, float* out);
void orc_prep_row(int32_t cols, const float* x, const uint8_t* sb, int8_t* q, float* scale, int32_t* sum8);
void orc_prep_slab(int32_t mc, int32_t cols, const float* x, const uint8_t* sb,
                   int8_t* xq_slab, float* scale, int32_t* sum8);
void orc_gemm_tiles(int32_t M, int32_t rows, int32_t cols, int32_t t0, int32_t t1,
                    const int8_t* xq, const float* xs, const int32_t* xsum,
                    const uint8_t* base, const uint64_t* offs, float* out, int skip_zero_blocks);
void orc_matmul_f32(int32_t M, int32_t rows, int32_t cols, int32_t n_tiles, const float* x,
                    const uint8_t* base, const uint64_t* offs, const uint8_t* sb, float* out);
void orc_embed(int32_t n_tokens, int32_t cols, const int32_t* ids, const uint8_t* base,
               const uint64_t* offs, const uint8_t* sb, float* out);
void orc_gemm_tiles_asym(int32_t is_had6, int32_t M, int32_t rows, int32_t cols, int32_t t0, int32_t t1,
                         const int8_t* xq, const float* xs, const int32_t* xsum,
                         const uint8_t* base, const uint64_t* offs, float* out);
void orc_matmul_asym_f32(int32_t is_had6, int32_t M, int32_t rows, int32_t cols, int32_t n_tiles,
                         const float* x, const uint8_t* base, const uint64_t* offs,
                         const uint8_t* sb, float* out);
void orc_embed_asym(int32_t is_had6, int32_t n_tokens, int32_t cols, const int32_t* ids,
                    const uint8_t* base, const uint64_t* offs, const uint8_t* sb, float* out);
void orc_embed_desc(const DpufWeightDesc* w, int32_t n_tokens, const int32_t* ids, float* out);
void orc_add_rmsnorm(int32_t n, float* x, const float* res, const float* w, float eps, float* out);
void orc_rope_tables(const DpufModelConfig* cfg, float* cos_tab, float* sin_tab);
void orc_rope_apply(int32_t hd, float* v, const float* c, const float* s);
void orc_attn_heads(int32_t hd, int32_t kv_len, float scale, const float* kc, const float* vc,
                    const float* q0, const float* q1, float* sc0, float* sc1, float* out0, float* out1);
float orc_swiglu1(float g, float u, float dz);
void orc_quant_q8(int32_t n, const float* src, int8_t* dst, float* scales);
void orc_attn_heads_q8(int32_t hd, int32_t kv_len, float scale, const int8_t* kq, const float* ks,
                       const int8_t* vq, const float* vs, const float* q0, const float* q1,
                       float* sc0, float* sc1, float* out0, float* out1);

OrcEngine* orc_engine_create(const DpufModelConfig* cfg, const DpufLayerWeights* layers,
                             const DpufWeightDesc* tok, const DpufWeightDesc* lm, const float* out_norm);
void orc_engine_destroy(OrcEngine* e);
int32_t orc_engine_set_slot(OrcEngine* e, int32_t s);
void orc_engine_reset_slot(OrcEngine* e, int32_t s);
int32_t orc_engine_freeze_prefix(OrcEngine* e, int32_t id, int32_t len);
int32_t orc_engine_apply_prefix(OrcEngine* e, int32_t slot, int32_t id);
int32_t orc_engine_set_kv(OrcEngine* e, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                          const float* k, const float* v);
int32_t orc_engine_get_kv(OrcEngine* e, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                          float* k, float* v);
void orc_engine_set_capture(OrcEngine* e, int32_t max_tokens);
const float* orc_engine_get_capture(OrcEngine* e);
int32_t orc_engine_forward(OrcEngine* e, int32_t n_tokens, const int32_t* ids, int32_t pos0,
                           const float* embeds_in, int32_t only_last, float* logits);
int32_t orc_argmax(const float* logits, int32_t V);
int32_t orc_top2_exit(const float* x, int32_t n, float thr);
int32_t orc_num_threads(void);
void orc_set_num_threads(int32_t n);
void orc_set_norm_order(int32_t tree);

#ifdef __cplusplus
}
#endif

#endif
