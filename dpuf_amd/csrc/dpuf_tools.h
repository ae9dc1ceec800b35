/*
 * dpuf_tools.h -- host tooling around the DPUF container for the MI355X build:
 * deterministic random-init weights, the mode 12 (Hadamard-4bit packed)
 * and mode 13 / 14 (asymmetric blk64 4 / 6-bit) packers, the .dpuf container writer, and the mmap reader that binds tensors
 * into DpufWeightDesc the way dpuf-cli.c does.  Plain C, no GPU code.
 */
#ifndef DPUF_TOOLS_H
#define DPUF_TOOLS_H

#include <stddef.h>
#include <stdint.h>
#include "../../include/dpuf_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    int32_t hidden_size;
    int32_t intermediate_size;
    int32_t num_layers;
    int32_t num_q_heads;
    int32_t num_kv_heads;
    int32_t head_dim;
    int32_t vocab_size;
    int32_t max_seq_len;
    int32_t tie_word_embeddings;
    float   weight_std;      /* N(0, weight_std) for every matrix */
    float   rms_eps;
    float   rope_theta;
    uint64_t seed;
    int32_t weight_plan;     /* 0: mode 12, shared Q/K/V and gate/up signs;
                                1: had4p-hybrid modes 13 / 14, signs per tensor */
} DpufToolsSpec;

typedef struct DpufToolsModel DpufToolsModel;

/* Deterministic N(0, std) weights: element i of tensor `name` depends only on
 * (seed, name, i), never on the thread count. */
DPUF_EXPORT void dpuf_tools_random_normal(float* out, size_t n, float std, uint64_t seed, const char* name);

/* fp32 -> bf16 (round to nearest even) -> fp32, in place. */
DPUF_EXPORT void dpuf_tools_round_bf16(float* x, size_t n);

/* fp32 <-> fp16 bit conversions (round to nearest even). */
DPUF_EXPORT uint16_t dpuf_tools_f32_to_f16(float f);
DPUF_EXPORT float dpuf_tools_f16_to_f32(uint16_t h);

/* Sign bits (cols/8 bytes) derived from a seed name. */
DPUF_EXPORT void dpuf_tools_sign_bits(uint8_t* out, int32_t cols, uint64_t seed, const char* sign_name);

/* Packs W[rows][cols] (fp32, taken as-is) into a mode 12 QR blob.
 * sign_bits: cols/8 bytes.  Returns a malloc'd blob, length in *len. */
DPUF_EXPORT uint8_t* dpuf_tools_pack_mode12(const float* W, int32_t rows, int32_t cols,
                                            const uint8_t* sign_bits, int32_t ecc_group,
                                            size_t* len);

/* Packs W into a mode 13 (bits 4) or mode 14 (bits 6) asymmetric blk64 QR
 * blob, weighted least-squares codes with weights (|w| + 1e-6)^w_pow (w_pow
 * <= 0: unweighted).  cols % 64 == 0.  Returns a malloc'd blob or NULL. */
DPUF_EXPORT uint8_t* dpuf_tools_pack_asym(const float* W, int32_t rows, int32_t cols, const uint8_t* sign_bits,
                                          int32_t ecc_group, int32_t bits, float w_pow, size_t* len);

/* Fills a DpufWeightDesc that points into a QR blob (no verification). */
DPUF_EXPORT int32_t dpuf_tools_bind_blob(const uint8_t* blob, size_t len, DpufWeightDesc* out);

/* RAW_TINY bf16 vector blob (10-byte header + bf16 data). */
DPUF_EXPORT uint8_t* dpuf_tools_pack_raw_tiny(const float* v, int32_t n, size_t* len);

/* Builds a whole random-init model in memory (Q/K/V and gate/up share signs). */
DPUF_EXPORT DpufToolsModel* dpuf_tools_build_model(const DpufToolsSpec* spec);

/* Writes the model as a .dpuf container; returns bytes written or 0. */
DPUF_EXPORT uint64_t dpuf_tools_save_container(const DpufToolsModel* m, const char* path);

/* mmaps a .dpuf container and binds it like dpuf-cli.c's dpuf_cli_open.
 * verify != 0 checks every tile's CRC32 and heals one bad tile per ECC group
 * into a heap copy.  *status: 0 ok, <0 error (see dpuf_tools.c). */
DPUF_EXPORT DpufToolsModel* dpuf_tools_open_container(const char* path, int32_t verify,
                                                      int32_t max_seq_len, int32_t* status);

DPUF_EXPORT void dpuf_tools_free_model(DpufToolsModel* m);

DPUF_EXPORT const DpufModelConfig* dpuf_tools_model_cfg(const DpufToolsModel* m);
DPUF_EXPORT const DpufLayerWeights* dpuf_tools_model_layers(const DpufToolsModel* m);
DPUF_EXPORT const DpufWeightDesc* dpuf_tools_model_tok(const DpufToolsModel* m);
DPUF_EXPORT const DpufWeightDesc* dpuf_tools_model_lm(const DpufToolsModel* m);
DPUF_EXPORT const float* dpuf_tools_model_out_norm(const DpufToolsModel* m);
DPUF_EXPORT int32_t dpuf_tools_model_healed(const DpufToolsModel* m);
DPUF_EXPORT uint64_t dpuf_tools_model_weight_bytes(const DpufToolsModel* m);

#ifdef __cplusplus
}
#endif

#endif
