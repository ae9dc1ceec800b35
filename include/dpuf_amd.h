/*
 * dpuf_amd.h -- entry points this build adds next to the dpuf_kernels.h ABI.
 * None of them has a counterpart in the reference; they exist for callers
 * that want device-side greedy sampling, for parity tests (per-layer residual
 * capture, KV injection) and for measurement.  The reference ABI does not
 * depend on any of them.
 */
#ifndef DPUF_AMD_H
#define DPUF_AMD_H

#include <stddef.h>
#include <stdint.h>
#include "dpuf_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Largest n_tokens a single forward call accepts (the reference caps at 256;
 * 512 is a compatible superset). */
#define DPUF_AMD_MAX_BATCH 512

/* 1 when a HIP device is usable, else 0. */
DPUF_EXPORT int32_t dpuf_amd_device_ok(void);

/* Text of the first HIP error recorded by the library ("" if none). */
DPUF_EXPORT const char* dpuf_amd_last_error(void);

/* forward_batch_ex plus greedy sampling on the device: *token_out receives the
 * first-max argmax (dpuf-cli.c:1997-2004 rule) of the last row's logits, so a
 * decode loop moves 4 bytes per token instead of V floats.  logits_out may be
 * NULL (no copy) or receive the last row's logits.  Same return codes as
 * dpuf_engine_forward_batch_ex. */
DPUF_EXPORT int32_t dpuf_amd_engine_forward_argmax(void* handle, int32_t n_tokens, const int32_t* token_ids,
                                                   int32_t pos0, const float* embeds_in, int32_t use_graph,
                                                   int32_t* token_out, float* logits_out);

/* Writes / reads positions [pos0, pos0+n) of (layer, kv head) of the active
 * slot, host pointers of n * head_dim floats.  0 ok, -1 bad arguments. */
DPUF_EXPORT int32_t dpuf_amd_engine_set_kv(void* handle, int32_t layer, int32_t kv_head, int32_t pos0, int32_t n,
                                           const float* k, const float* v);
DPUF_EXPORT int32_t dpuf_amd_engine_get_kv(void* handle, int32_t layer, int32_t kv_head, int32_t pos0, int32_t n,
                                           float* k, float* v);

/* Captures the residual stream after every layer ([num_layers][n][hidden])
 * for calls with n_tokens <= max_tokens (0 disables).  get_capture copies
 * num_layers * max_tokens * hidden floats.  0 ok, -1 error. */
DPUF_EXPORT int32_t dpuf_amd_engine_set_capture(void* handle, int32_t max_tokens);
DPUF_EXPORT int32_t dpuf_amd_engine_get_capture(void* handle, float* out, size_t n_floats);

/* Kernel timing with HIP events on the engine's stream.  Kinds:
 * 0 gate/up GEMV, 1 down GEMV, 2 QKV GEMV, 3 O GEMV, 4 LM head, 5 attention,
 * 6 norm+prep, 7 whole forward call.  get_timing returns total ms, launch
 * count and algorithmic bytes for a kind; enabling resets the counters. */
DPUF_EXPORT void dpuf_amd_engine_set_timing(void* handle, int32_t enable);
DPUF_EXPORT int32_t dpuf_amd_engine_get_timing(void* handle, int32_t kind, double* total_ms, int64_t* count,
                                               double* bytes);

/* Graph replay of one-token steps, on by default: the reference entry points
 * and dpuf_amd_engine_forward_argmax (use_graph set) replay a HIP graph
 * captured once per step shape.  0 enqueues every kernel of every step
 * instead (for per-kernel traces) and releases the graphs kept so far. */
DPUF_EXPORT void dpuf_amd_engine_set_graphs(void* handle, int32_t enable);

/* Mode 12 tile bytes resident in HBM (all layers + LM head). */
DPUF_EXPORT uint64_t dpuf_amd_engine_weight_bytes(void* handle);

/* Number of forward calls in which the LM-head early exit fired. */
DPUF_EXPORT int64_t dpuf_amd_engine_early_exit_count(void* handle);

/* Attention launches enqueued so far in this process, by path (which: 0 the
 * prefill split kernels with the register-tiled softmax + P.V, 1 the
 * one-token long-context kernels (scores, softmax once per row, wide P.V),
 * 2 the split scores + LDS softmax / P.V kernels, 3 the one-pair-per-workgroup
 * fallback, 4 the fused short-context decode kernel, 5 the int8-cache
 * kernels); -1 for another `which`.  Enqueued, not executed: a replayed graph
 * counts at its capture only.  For tests that check which path a shape
 * takes. */
DPUF_EXPORT int64_t dpuf_amd_attn_path_count(int32_t which);

/* Times `iters` back-to-back launches of one GEMV kind over resident weights
 * (which: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down, 7 LM head, 8 gate+up as
 * one launch, 9 q+k+v as one launch), cycling through layers
 * start..num_layers-1 so that consecutive launches read distinct weights.
 * Returns the mean ms per launch (or < 0 on error); *bytes gets the
 * algorithmic bytes of one launch (weight groups + activations + outputs). */
DPUF_EXPORT double dpuf_amd_gemv_bench(void* handle, int32_t which, int32_t M, int32_t iters, int32_t start_layer,
                                       double* bytes);

/* Copies `bytes` between two device buffers `iters` times (hipMemcpyAsync
 * device to device) and returns the mean ms per copy; a reference of known
 * traffic for calibrating hardware byte counters.  < 0 on error. */
DPUF_EXPORT double dpuf_amd_copy_bench(size_t bytes, int32_t iters);

/* Caps the workgroups of an M = 1 GEMV launch at n (n <= 0: no cap beyond
 * what the device holds at once), process-wide.  A smaller cap gives each
 * workgroup more 8-row groups to walk; results do not depend on it.  For
 * tests of the multi-group path and for tuning. */
DPUF_EXPORT void dpuf_amd_set_gemv_max_workgroups(int32_t n);

/* Runs the device logit reductions on n host floats placed `offset` floats
 * (0..3) past a 16-byte boundary: mode 1 returns the first-maximum index the
 * greedy sampler takes (dpuf-cli.c:1997-2004); mode 0 returns the Zone-A
 * early-exit flag, 1 when thr > 0 and top1 - top2 >= thr over the multiset
 * (dpuf_engine.c:2101-2110).  -1 on error.  For tests. */
DPUF_EXPORT int32_t dpuf_amd_reduce_check(const float* x, int32_t n, int32_t offset, int32_t mode, float thr);

/* dpuf_amd_reduce_check without allocating: the reduction of n floats
 * already in device memory (d_x) into one int32 in device memory (d_out),
 * enqueued on hip_stream (a hipStream_t; NULL is the default stream) without
 * synchronising.  mode and thr as in dpuf_amd_reduce_check.  The partials
 * live in a 512-byte array of the library's that each device holds until the
 * process ends; every call on a device shares it, so calls that overlap on
 * one device (two streams, two threads) race and must be serialised by the
 * caller.  n is at most DPUF_AMD_NOALLOC_MAX_N.  Returns 0 when enqueued, -1
 * bad pointer or mode, -2 n out of range, -6 device error
 * (dpuf_amd_last_error says which).
 * No counterpart in the reference: for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc -- and sample the greedy token on the device. */
#define DPUF_AMD_NOALLOC_MAX_N (1 << 30)
DPUF_EXPORT int32_t dpuf_amd_reduce_check_noalloc(const float* d_x, int32_t n, int32_t mode, float thr,
                                                  int32_t* d_out, void* hip_stream);

/* One next token for each of n sessions in one pass (serving several
 * conversations with one read of the weights): token_ids[i] is appended to
 * KV slot slot_ids[i] (distinct slots, allocated on demand) at positions[i]
 * (any position below max_seq_len, for either KV cache type); logits_out
 * [n][V] and/or tokens_out [n] (greedy ids), in the caller's order.  Per token
 * the results equal a one-token dpuf_engine_forward_batch on that slot (decode
 * keep-tiles setting, no Zone-A early exit).  The projections and the LM head
 * run once for all n tokens; the attention of sessions with at most 192 keys
 * (fp32 cache) is one launch, every other session's takes the one-token
 * launches of its own length.  0 on success; -1 bad arguments or a repeated
 * slot, -2 above DPUF_AMD_MAX_BATCH or out of memory, -3 position out of
 * range, -4 token id out of range, -5 head dim other than 64/128/256, -6
 * device error.  No counterpart in the reference,
 * whose forward serves one slot per call; for serving loops (dpuf-cli.c's
 * one-slot-per-call generation stays as it is). */
DPUF_EXPORT int32_t dpuf_amd_engine_forward_slots(void* handle, int32_t n, const int32_t* slot_ids,
                                                  const int32_t* token_ids, const int32_t* positions,
                                                  float* logits_out, int32_t* tokens_out);

/* dpuf_qr_verify_tiles_ex (reference dpuf_avx2.c:846-908) with the CRC32 of
 * every tile body computed on the GPU: same arguments, tile_ok_out and return
 * value (the number of bad tiles; -1 on error).  No counterpart in the
 * reference, which checks tiles on the CPU while binding tensors; for hosts
 * that verify multi-GB files before dpuf_engine_create. */
DPUF_EXPORT int32_t dpuf_amd_verify_tiles_device(int32_t mode, int32_t n_tiles, int32_t cols,
                                                 const uint8_t* tensor_base, const uint64_t* tile_offsets,
                                                 uint8_t* tile_ok_out);

#ifdef __cplusplus
}
#endif

#endif
