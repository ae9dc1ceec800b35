/*
 * hip_layer.h -- the thin C ABI between the C host engine (engine.c) and the
 * gfx950 HIP code (rt.hip, gemv.hip, gemm.hip, attn.hip, attn_wide.hip,
 * attn_dec.hip).  Plain pointers and sizes only; every
 * function that launches work takes the engine's stream as an opaque handle.
 */
#ifndef DPUF_HIP_LAYER_H
#define DPUF_HIP_LAYER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One mode 12, 13 or 14 matrix resident in HBM in the row-block layout
 * written by dpuf_hip_relayout: group g (rows 8g .. 8g+7) at
 * g + g * (cols/32) * U (U = 144, or 208 for mode 14), holding [cols/32][8]
 * fp16 scales (mode 12: the 32-block scales; modes 13 / 14: d of 64-block j
 * as "block" 2j, m as 2j+1), then per 32-column block 8 rows x 16 bytes of
 * nibbles (row ri's four .dpuf chunk words of the block, in chunk order),
 * and for mode 14 per block 8 rows x 8 bytes of bits 4..5: word w, byte k
 * holds chunk 2w's columns +k and +4+k in bits 0-1 and 2-3, chunk 2w+1's in
 * bits 4-5 and 6-7. */
typedef struct {
    const uint8_t*  g;
    const uint8_t*  sign;
    int32_t rows, cols, n_groups;
    int32_t mode;   /* 12, 13 or 14 */
} DpufDevW;

/* Bytes of one 8-row group per 32 columns in .dpuf tiles and on the device. */
static inline int32_t dpuf_grp_unit(int32_t mode) { return mode == 14 ? 208 : 144; }

/* Prepped activations of M rows: q int8 [M][K], s f32 [M][K/32], m i32 [M][K/32],
 * and h, the same q as fp16 [M][K] (the M > 1 GEMM's input; the prep
 * kernels fill it when non-NULL and M > 1). */
typedef struct {
    int8_t*  q;
    float*   s;
    int32_t* m;
    uint16_t* h;
} DpufPrep;

/* One layer's int8 KV cache (kv_type 1): K and V [n_kv][max_seq][hd] int8
 * with per-32-column scales [n_kv][max_seq][hd / 32]. */
typedef struct {
    int8_t* kq;
    int8_t* vq;
    float* ks;
    float* vs;
} DpufKvQ8;

/* A cache warm-up by otherwise idle workgroups of a latency-bound launch:
 * they read weight groups that later one-row GEMVs stream, on the XCD whose
 * workgroups will read them (a GEMV's workgroup b runs on XCD b % 8), so
 * those reads hit the XCD's L2 or the Infinity Cache instead of waiting on
 * HBM.  Job j: group g (of n_groups, group_bytes each, from p) is read by its
 * GEMV's workgroup wb + g % nwg in round g / nwg; rounds [r0, r0 + nr) are
 * warmed.  n_wg warm-up workgroups (a multiple of 8; the launcher sets it);
 * sink: a device word written only when the bytes hash to one value, so the
 * reads are kept. */
#define DPUF_WARM_JOBS 6
typedef struct {
    const uint8_t* p;
    int32_t n_groups, group_bytes, wb, nwg, r0, nr;
} DpufWarmJob;
typedef struct {
    DpufWarmJob j[DPUF_WARM_JOBS];
    int32_t n_jobs;
    int32_t n_wg;
    int32_t* sink;
} DpufWarm;

/* One matrix of a fused GEMV launch: groups [g0, g1) of w, reading prep p,
 * writing out[m * ldo + row]. */
typedef struct {
    DpufDevW w;
    int32_t g0, g1;
    DpufPrep p;
    float* out;
    int32_t ldo;
} DpufGemvJob;

int32_t dpuf_hip_device_count(void);
const char* dpuf_hip_error_string(void);
int32_t dpuf_hip_ok(void);          /* 1 if no HIP error has been recorded */
void dpuf_hip_clear_error(void);

void* dpuf_hip_malloc(size_t bytes);
void  dpuf_hip_free(void* p);
void* dpuf_hip_host_alloc(size_t bytes);   /* pinned */
/* pinned and fine-grained: kernels read and write it directly, the host sees
 * their stores once the stream has drained */
void* dpuf_hip_host_alloc_io(size_t bytes);
void  dpuf_hip_host_free(void* p);
void* dpuf_hip_stream_create(void);
void  dpuf_hip_stream_destroy(void* s);
int32_t dpuf_hip_sync(void* s);
void dpuf_hip_h2d(void* dst, const void* src, size_t n, void* s);
void dpuf_hip_d2h(void* dst, const void* src, size_t n, void* s);
void dpuf_hip_d2d(void* dst, const void* src, size_t n, void* s);
void dpuf_hip_fill_zero(void* dst, size_t n, void* s);   /* kernel fill, graph-safe */
void dpuf_hip_fill_f32(float* dst, size_t n, float v, void* s);

void* dpuf_hip_event_create(void);
void  dpuf_hip_event_destroy(void* e);
void  dpuf_hip_event_record(void* e, void* s);
float dpuf_hip_event_elapsed_ms(void* a, void* b);   /* synchronises on b */
void  dpuf_hip_event_sync(void* e);                  /* waits for the work before e */

/* Graph capture of a stream into a replayable executable graph. */
int32_t dpuf_hip_capture_begin(void* s);
void* dpuf_hip_capture_end(void* s);                 /* returns exec graph or NULL */
int32_t dpuf_hip_graph_launch(void* g, void* s);
void dpuf_hip_graph_destroy(void* g);

/* Kernels.  pos0 is read from device memory so a captured step replays at
 * any position.  Rows with a negative id take their hidden state from embeds,
 * which is fine-grained host memory when emb_host is set. */
void dpuf_hip_embed(void* s, DpufDevW w, const int32_t* ids, int32_t M, const float* embeds, int32_t emb_host,
                    float* out, const int32_t* pos_src, int32_t* pos_dst, int32_t* serial_dst);
/* host[0..3) = {flag_valid ? words[0] : 0, words[1], words[2]} (words: the
 * device's early-exit flag, argmax token, error word) */
void dpuf_hip_publish(void* s, const int32_t* words, int32_t flag_valid, int32_t* host);
/* The one-row GEMV of job (as dpuf_hip_gemv with M = 1) whose chains also
 * write partials of the LM-head reductions (top-2 and first maximum of the
 * rows each computed; 16 bytes each) to red; returns their count (-1 on an
 * error, including more than red_cap).  With skip_flag set the rows are
 * filled and no partial is written. */
int32_t dpuf_hip_gemv_red(void* s, const DpufGemvJob* job, const int32_t* skip_flag, float fill, void* red,
                          int32_t red_cap);
/* One workgroup over the zone rows' n partials: *flag = the early-exit test
 * (thr > 0 and top-1 - top-2 >= thr), zone (16 bytes) = their merge. */
void dpuf_hip_lm_zone(void* s, const void* part, int32_t n, float thr, int32_t* flag, void* zone);
/* One workgroup: the first maximum of the row from n partials (with zone:
 * the zone's merge plus, when words[0] is set, the fill value from row
 * fill_row on instead of the partials), 0 when *x0 is NaN; writes it to
 * words[1] and publishes words as dpuf_hip_publish does. */
void dpuf_hip_lm_argmax_publish(void* s, const void* part, int32_t n, const void* zone, float fill, int32_t fill_row,
                                const float* x0, int32_t* words, int32_t flag_valid, int32_t* host);
/* h_out = h + res for M rows of H (res NULL: no add, h_out unused), then
 * the RMSNorm of that sum (of h when res is NULL) with weights w and the
 * prep of the result for each of the n_prep sign vectors into preps[i] (and
 * into xn_out when non-NULL).  h_out may equal h, at the cost of the
 * one-workgroup-per-row form. */
void dpuf_hip_resnorm_prep(void* s, int32_t M, int32_t H, const float* h, const float* res, float* h_out,
                           const float* w, float eps, int32_t n_prep, const uint8_t* const* signs,
                           const DpufPrep* preps, float* xn_out);
void dpuf_hip_prep(void* s, int32_t M, int32_t K, const float* x, const uint8_t* sign, DpufPrep p);
void dpuf_hip_swiglu_prep(void* s, int32_t M, int32_t I, const float* gate, const float* up,
                          float dz, const uint8_t* sign, DpufPrep p);
/* M == 1: SwiGLU + prep of gate / up [I] (up NULL: the plain prep of gate)
 * and the GEMV of job over it in one launch; the producing workgroups set
 * flags[0 .. 512) entries to the step
 * serial *serial (device memory, a value new to these flags).  -1: the plan
 * does not allow it (nothing launched; use the two calls above). */
int32_t dpuf_hip_swiglu_gemv(void* s, int32_t I, const float* gate, const float* up, float dz, const uint8_t* sign,
                             const DpufGemvJob* job, int32_t* flags, const int32_t* serial);
/* .dpuf tile region of a mode 12 / 13 / 14 matrix (tile t at src + offs[t])
 * -> row-block layout. */
void dpuf_hip_relayout(void* s, const uint8_t* src, const uint64_t* offs, int32_t n_groups, int32_t n_blk,
                       int32_t mode, uint8_t* dst);
/* M == 1: GEMV of up to three matrices sharing K, with the activations of
 * each job in jobs[i].p; a non-NULL skip_flag that reads non-zero makes the
 * launch write `fill` to every row instead.  M > 1: the slab GEMM. */
void dpuf_hip_gemv(void* s, int32_t M, int32_t n_jobs, const DpufGemvJob* jobs,
                   const int32_t* skip_flag, float fill);
/* One GEMV job that also sets rows [r0, r1) of job->out to 0 (every token
 * row): for M > 1 inside the GEMM launch, for M == 1 with a second launch. */
void dpuf_hip_gemv_zero(void* s, int32_t M, const DpufGemvJob* job, int32_t r0, int32_t r1);
/* Appends to wm the rounds [r0, r0 + nr) of the one-row GEMV over these
 * jobs (one mode) as the GEMV will be launched; returns 0 when they do not
 * fit (wm unchanged). */
int32_t dpuf_hip_warm_add(DpufWarm* wm, int32_t n_jobs, const DpufGemvJob* jobs, int32_t r0, int32_t nr);
/* Producer workgroups ahead of the GEMV workgroups in dpuf_hip_swiglu_gemv's
 * launch of job over I activations (0 when that launch does not apply):
 * what a warm-up plan of the job adds to its workgroup base. */
int32_t dpuf_hip_fed_producers(int32_t I, const DpufGemvJob* job);
/* gate and up (jobs[0], jobs[1]) of M tokens and the SwiGLU + dead zone dz +
 * prep (sign bits of the down input) of their result into out, in one
 * launch; -1 with nothing launched when the shapes do not take it (then
 * dpuf_hip_gemv + dpuf_hip_swiglu_prep).  out must not be the jobs' input. */
int32_t dpuf_hip_gemm_swiglu(void* s, int32_t M, const DpufGemvJob* jobs, float dz, const uint8_t* sign,
                             DpufPrep out);
/* The same for 2 .. 8 tokens on the few-token kernel (gate and up as the
 * two fragments of its pairs); -1 with nothing launched when the shapes do
 * not take it. */
int32_t dpuf_hip_mvt_swiglu(void* s, int32_t M, const DpufGemvJob* jobs, float dz, const uint8_t* sign,
                            DpufPrep out);
/* Caps the workgroups of an M == 1 GEMV or K-split GEMM launch (<= 0:
 * device capacity only). */
void dpuf_hip_set_gemv_max_wg(int32_t n);
/* Device word (4 bytes, zero) that the GEMV kernels of this thread's
 * following launches set non-zero when a bounded wait runs out; the caller
 * reads it after synchronising.  M == 1 GEMV launches fail without one. */
void dpuf_hip_bind_error_word(int32_t* d_word);
void dpuf_hip_qk_rope_kv(void* s, int32_t M, float* q, float* k, const float* v,
                         const float* q_norm, const float* k_norm, float eps,
                         const float* cos_tab, const float* sin_tab, float* kc, float* vc,
                         const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                         const DpufKvQ8* c8);
/* With c8 set, K (after QK-norm and RoPE) and V go into the int8 cache
 * instead of kc / vc. */
void dpuf_hip_attn(void* s, int32_t M, const float* q, const float* kc, const float* vc, float* out,
                   float* scores, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd,
                   int32_t max_seq, float scale);
/* Split attention (scores kernel + softmax/P.V kernel) over keys up to
 * lmax; -1 (nothing launched) when the shape does not fit.  With op.q and
 * prepped set, a launch that can also writes the O projection's input prep
 * (signs o_sign) in place of `out` and sets *prepped to 1. */
int32_t dpuf_hip_attn_split(void* s, int32_t M, int32_t lmax, const float* q, const float* kc, const float* vc,
                            float* out, float* scores, const int32_t* pos0p, int32_t n_q, int32_t n_kv, int32_t hd,
                            int32_t max_seq, float scale, const uint8_t* o_sign, DpufPrep op, int32_t* prepped);
/* One-token decode past the fused kernel's range (the split path's wide
 * kernels) with the QK-norm, RoPE and KV store of the token (raw q, k, v)
 * done inside the scores launch; -1 with nothing launched when that path
 * does not apply (then qk_rope_kv + attn_split).  warm (or NULL): weight
 * groups that workgroups of the P.V launch read into the caches on the CUs
 * its chains leave idle (groups of 2 and 4). */
int32_t dpuf_hip_attn_decode_rope(void* s, int32_t lmax, float* q, const float* k, const float* v, const float* qn,
                                  const float* kn, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                                  float* vc, float* out, float* scores, const int32_t* pos0p, int32_t n_q,
                                  int32_t n_kv, int32_t hd, int32_t max_seq, float scale, const DpufWarm* warm);
/* Attention over the int8 KV cache (kv_type 1) for M tokens at positions
 * pos0 .. pos0 + M - 1 of one layer; lmax bounds the keys any replay reaches.
 * warm (or NULL): as for dpuf_hip_attn_decode_rope, on the one-token path. */
void dpuf_hip_attn_q8(void* s, int32_t M, int32_t lmax, const float* q, DpufKvQ8 c8, float* out, float* scores,
                      const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq, float scale,
                      const DpufWarm* warm);
/* n rows of fp32 K and V (device) quantised into rows row0 .. of the int8
 * cache, as the KV store does; and n values from element off dequantised. */
void dpuf_hip_q8_rows(void* s, const float* k, const float* v, int32_t n, int32_t hd, DpufKvQ8 c8, size_t row0);
void dpuf_hip_q8_dequant(void* s, DpufKvQ8 c8, size_t off, size_t n, float* k, float* v);
/* Keys the fused decode attention takes (positions 0 .. 191); longer
 * contexts go to the split kernels. */
#define DPUF_HIP_DEC_MAX_KEYS 192
/* One-token-per-session fused QK-norm + RoPE + KV store + attention +
 * O-input prep for M tokens: token m at position pos0[m] (pos0[m] <
 * DPUF_HIP_DEC_MAX_KEYS, checked by the caller: the position is read on the
 * device); with kcs / vcs set (device arrays of M session KV-cache bases,
 * plus l_off floats) each token uses its own session's cache, otherwise all
 * use kc / vc.  Returns -1 (nothing launched) for head dims other than 64,
 * 128, 256. */
int32_t dpuf_hip_attn_dec(void* s, int32_t M, const float* q, const float* k, const float* v, const float* q_norm,
                          const float* k_norm, float eps, const float* cos_tab, const float* sin_tab, float* kc,
                          float* vc, const int32_t* pos0, int32_t n_q, int32_t n_kv, int32_t hd, int32_t max_seq,
                          float scale, float* ao, const uint8_t* o_sign, DpufPrep op, float* const* kcs,
                          float* const* vcs, size_t l_off, DpufWarm warm);
/* Attention launches enqueued per path (dpuf_amd_attn_path_count); -1 for
 * another `which`. */
#define DPUF_HIP_ATTN_PATHS 6
int64_t dpuf_hip_attn_path_count(int32_t which);
void dpuf_hip_zero_rows(void* s, int32_t M, float* out, int32_t ld, int32_t r0, int32_t r1);
/* CRC32 of n tile bodies (base + off[t], len[t] bytes) against want[t]: ok[t] = 1 when equal. */
void dpuf_hip_crc_tiles(void* s, const uint8_t* base, const uint64_t* off, const uint32_t* len,
                        const uint32_t* want, uint8_t* ok, int32_t n);
void dpuf_hip_capture(void* s, int32_t M, int32_t H, const float* h, const float* hn, float* cap);
/* Device reductions of a logit row (two launches each); scratch holds
 * DPUF_HIP_RED_SCRATCH bytes of partials. */
#define DPUF_HIP_RED_SCRATCH 512
void dpuf_hip_topcheck(void* s, const float* logits, int32_t n, float thr, int32_t* flag, void* scratch);
void dpuf_hip_argmax(void* s, const float* logits, int32_t V, int32_t* out, void* scratch);
/* The first-max argmax of n rows of V logits (rows V apart) into out[0..n)
 * and, when host is set, host[0..n) (fine-grained host memory); scratch
 * holds n x 512 bytes of partials. */
void dpuf_hip_argmax_rows(void* s, const float* logits, int32_t V, int32_t n, int32_t* out, int32_t* host,
                          void* scratch);
/* The same reductions with the partials in the library's own file-scope
 * device array (one per device, RED_NB float2): no allocation.  mode 1
 * argmax, 0 top-2 check.  Concurrent calls on one device share the array.
 * 0 ok, -6 when the array's address or the launch failed. */
int32_t dpuf_hip_reduce_noalloc(const float* x, int32_t n, int32_t mode, float thr, int32_t* out, void* s);
void dpuf_hip_fwht_sign(void* s, int32_t M, int32_t K, const float* x, const uint8_t* sign, float* out);
void dpuf_hip_slab_pack(void* s, int32_t mc, int32_t K, DpufPrep rows, int32_t* sq, float* ss, int32_t* sm);
void dpuf_hip_slab_unpack(void* s, int32_t M, int32_t K, const int32_t* sq, const float* ss, const int32_t* sm,
                          DpufPrep rows);

#ifdef __cplusplus
}
#endif

#endif
