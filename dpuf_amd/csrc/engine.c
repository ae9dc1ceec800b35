/*
 * engine.c -- host side of the MI355X DPUF engine (C11).
 *
 * Implements the dpuf_engine_* ABI of include/dpuf_kernels.h over the thin
 * HIP layer of hip_layer.h.  The structure follows the reference engine
 * (dpuf_engine.c in dulePan/dpuf): create copies the config and layer
 * descriptors (dpuf_engine.c:1208-1354), forward runs embed -> L x [norm,
 * QKV, rope+KV, attention, O, norm, gate/up, SwiGLU, down] -> norm -> LM head
 * (dpuf_engine.c:1625-2147).  What changes is where the work happens: every
 * weight payload is validated and uploaded to HBM once at create, and each
 * step of the loop is one HIP kernel launch on the engine's stream.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/dpuf_amd.h"
#include "../../include/dpuf_kernels.h"
#include "hip_layer.h"

#define N_SLOTS 8
#define N_GRAPHS 8  /* captured one-token steps kept per engine */
#define LM_RED_CAP 16384 /* LM-head partials (chains of one GEMV launch); also the row argmax scratch */
#define N_PREFIX 8
#define N_KINDS 8
#define MAX_EVENTS 8192

enum { K_GU = 0, K_DOWN, K_QKV, K_O, K_LM, K_ATTN, K_PREP, K_CALL };
enum { W_Q = 0, W_K, W_V, W_O, W_GATE, W_UP, W_DOWN };

typedef struct {
    const uint8_t* host_base;
    void* d_groups;   /* row-block layout, n_groups * (cols/32) * 144 bytes */
    void* d_sign;
    uint64_t bytes;
} Upload;

typedef struct {
    DpufModelConfig cfg;
    int32_t L, H, I, nq, nkv, hd, qd, kvd, V, max_seq;
    DpufDevW* lw;        /* [L][7] */
    float** d_norm;      /* [L][4]: attn, q, k, ffn */
    DpufDevW tok, lm;
    float* d_out_norm;
    float* d_cos;
    float* d_sin;
    /* KV cache arrays per slot and per frozen prefix, [L][n_kv][positions]
     * rows of kv_row[i] bytes: fp32 K, V (kv_type 0), or int8 K, V and their
     * per-32 fp32 scales (kv_type 1, dpuf_engine.c:1182-1206) */
    int32_t kv_n;
    size_t kv_row[4];
    void* kv[N_SLOTS][4];
    int32_t active;
    void* pkv[N_PREFIX][4];
    int32_t plen[N_PREFIX], pcap[N_PREFIX], pvalid[N_PREFIX];
    /* scratch for up to DPUF_AMD_MAX_BATCH rows */
    float *h, *hn, *q, *k, *v, *ao, *gate, *up, *logits, *scores, *embeds, *capture;
    /* the residual stream alternates between h and h2: each residual add
     * reads one and writes the other (its kernel's workgroups all read the
     * old stream); hcur is the current one while a step is enqueued */
    float *h2, *hcur;
    int32_t capture_cap;
    DpufPrep prep[3];
    int32_t *d_ids, *d_pos0, *d_flag, *d_tok, *d_err;
    /* step serial: the host numbers every forward call (h_io[IO_POS + 1]),
     * the embedding kernel copies it to d_serial; d_pflag [L][2][512] are
     * the producer flags of the one-row launches that prep their own input
     * (O projection: slot 0, down projection: slot 1), which take the serial
     * of the step that set them (never reset) */
    int32_t *d_serial, *d_pflag;
    int32_t serial;
    void* d_red; /* partials of the device argmax / top-2 reductions */
    /* LM-head partials written by the one-row LM-head GEMV's chains
     * (LM_RED_CAP of 16 bytes), then the Zone-A merge (16 bytes) */
    void* d_lmred;
    /* one token per session (dpuf_amd_engine_forward_slots): while ms_n > 0
     * the layers run ms_n tokens, token m of slot ms_slot[m] at position
     * ms_pos[m] (device copy d_ms_pos); the first ms_short of them (fp32
     * cache, at most DPUF_HIP_DEC_MAX_KEYS keys) through one fused decode
     * attention launch with the KV caches at d_ms_kc[m] / d_ms_vc[m], every
     * other one through the one-token attention launches of its own slot */
    int32_t ms_n, ms_short;
    int32_t ms_slot[DPUF_AMD_MAX_BATCH], ms_pos[DPUF_AMD_MAX_BATCH];
    int32_t *d_ms_pos, *d_ms_tok;
    float **d_ms_kc, **d_ms_vc;
    int32_t* h_pinned;   /* host staging: [3] error word of the GEMV bench */
    /* fine-grained host memory the kernels use directly (no copies): h_io
     * holds a step's ids [0, B), its pos0 at IO_POS (read by the embedding
     * kernel) and the published flag, token and error word at IO_OUT;
     * h_logits receives the one LM-head row of a step whose logits go to the
     * host (written by the GEMV itself); h_emb takes the hidden state of a
     * one-row embeds_in step, read there by the embedding kernel */
    int32_t* h_io;
    float* h_logits;
    float* h_emb;
    /* multi-session steps: the pinned staging of the per-session tables,
     * laid out as on the device (B cache bases of K, B of V, then B
     * positions: one copy), and the next tokens, which the argmax kernel
     * writes to this fine-grained host array itself */
    void* h_ms;
    int32_t* h_tok;
    uint8_t* q_idx;      /* per layer: prep index of q,k,v (3 bytes) and gate/up (2 bytes) */
    float deadzone;
    void* stream;
    Upload* ups;
    int32_t n_ups;
    uint64_t weight_bytes;
    int64_t early_exits;
    /* timing */
    int32_t timing;
    void* ev[MAX_EVENTS];
    int32_t ev_kind[MAX_EVENTS / 2];
    double ev_bytes[MAX_EVENTS / 2];
    int32_t n_ev;
    double t_ms[N_KINDS];
    int64_t t_cnt[N_KINDS];
    double t_bytes[N_KINDS];
    /* one-token steps captured as HIP graphs, one per key (only_last, keep
     * tiles, early tiles, slot, margin, attention key bucket, argmax); a
     * graph replays at every position of its bucket (attn_bucket): a host
     * that alternates slots or entry points keeps its graphs; the least
     * recently used one makes room */
    void* graphs[N_GRAPHS];
    int32_t graph_keys[N_GRAPHS][7];
    uint32_t graph_used[N_GRAPHS];
    uint32_t graph_tick;
    int32_t no_graphs; /* dpuf_amd_engine_set_graphs(0) */
    /* the forward being enqueued: host copy of pos0, and whether it is being
     * captured into a graph that replays at every position of the key bucket
     * cap_lmax (the largest key count the captured attention launches serve) */
    int32_t host_pos0;
    int32_t capturing;
    int32_t cap_lmax;
} Engine;

#define IO_POS DPUF_AMD_MAX_BATCH
#define IO_OUT (DPUF_AMD_MAX_BATCH + 4)

/* Decode attention switches from the fused short-context kernel to the split
 * (scores + softmax/P.V) kernels once kv_len exceeds this. */
#define ATT_SPLIT_MIN DPUF_HIP_DEC_MAX_KEYS

/* Key bucket of a captured one-token step that attends over `keys` keys: the
 * fused kernel's range as one bucket, then 256, 512, 1024 and multiples of
 * 1024 (at most max_seq).  The captured attention launches are sized for the
 * bucket's top, so they take the path, and about the launch shapes, of an
 * eager step at that many keys, whatever max_seq is; a longer context
 * captures the next bucket (at most one capture per 1024 decoded tokens). */
static int32_t attn_bucket(const Engine* e, int32_t keys) {
    int32_t b;
    if (keys <= ATT_SPLIT_MIN) b = ATT_SPLIT_MIN;
    else if (keys <= 1024) for (b = 256; b < keys; b <<= 1) {}
    else b = (keys + 1023) & ~1023;
    return b < e->max_seq ? b : e->max_seq;
}

/* ------------------------------------------------------------------------- */

static int env_int(const char* name, int* out) {
    const char* s = getenv(name);
    if (!s) return 0;
    *out = atoi(s);
    return 1;
}

/* Start of every entry point that launches work: a fresh per-call error
 * state, and the engine's device error word for the GEMV kernels. */
static void begin_call(Engine* e) {
    dpuf_hip_clear_error();
    dpuf_hip_bind_error_word(e->d_err);
}

/* After the stream has drained: 0 when neither the runtime nor a kernel
 * (through the device error word, already copied to *word) reported a
 * failure; else the word is cleared for the next call and -6 returned. */
static int32_t end_call(Engine* e, int32_t word) {
    if (word != 0) {
        dpuf_hip_fill_zero(e->d_err, 4, e->stream);
        dpuf_hip_sync(e->stream);
        return -6;
    }
    return dpuf_hip_ok() ? 0 : -6;
}

/* Starts a timed region: reserves an event pair, records its start and
 * returns its index (-1 when timing is off or the table is full).  Regions
 * may nest (the whole-call region encloses the per-kernel ones). */
static int tm_begin(Engine* e, int kind, double bytes) {
    if (!e->timing || e->n_ev + 2 > MAX_EVENTS) return -1;
    const int i = e->n_ev;
    if (!e->ev[i]) e->ev[i] = dpuf_hip_event_create();
    if (!e->ev[i + 1]) e->ev[i + 1] = dpuf_hip_event_create();
    if (!e->ev[i] || !e->ev[i + 1]) return -1;
    e->ev_kind[i / 2] = kind;
    e->ev_bytes[i / 2] = bytes;
    e->n_ev += 2;
    dpuf_hip_event_record(e->ev[i], e->stream);
    return i;
}

static void tm_end(Engine* e, int i) {
    if (i < 0) return;
    dpuf_hip_event_record(e->ev[i + 1], e->stream);
}

static void tm_collect(Engine* e) {
    if (!e->timing) return;
    for (int32_t i = 0; i < e->n_ev; i += 2) {
        int k = e->ev_kind[i / 2];
        e->t_ms[k] += dpuf_hip_event_elapsed_ms(e->ev[i], e->ev[i + 1]);
        e->t_cnt[k] += 1;
        e->t_bytes[k] += e->ev_bytes[i / 2];
    }
    e->n_ev = 0;
}

static int mode_ok(int32_t mode) {
    return mode == DPUF_MODE_QR_HAD4_PACKED || mode == DPUF_MODE_QR_HAD4_ASYM || mode == DPUF_MODE_QR_HAD6;
}

/* Checks that every tile of a mode 12, 13 or 14 descriptor lies inside its
 * payload and that row counts are consistent, so that no kernel can read out
 * of bounds. */
static int validate_desc(const DpufWeightDesc* d) {
    if (!d || !mode_ok(d->mode)) return 0;
    if (d->rows <= 0 || d->cols <= 0 || (d->cols % 64) != 0 || d->n_tiles != (d->rows + 15) / 16) return 0;
    if (!d->tensor_base || !d->tile_offsets) return 0;
    const uint64_t total = d->tile_offsets[d->n_tiles];
    const uint64_t grp = (uint64_t)(d->cols / 32) * (uint64_t)dpuf_grp_unit(d->mode);
    for (int32_t t = 0; t < d->n_tiles; t++) {
        uint64_t o = d->tile_offsets[t];
        if (o % 16 != 0 || o + 16 > total) return 0;
        if (t > 0 && o <= d->tile_offsets[t - 1]) return 0; /* tiles in file order */
        DpufQrTileHdr th;
        memcpy(&th, d->tensor_base + o, sizeof th);
        int32_t want = (t * 16 + 16 <= d->rows) ? 16 : d->rows - t * 16;
        if (th.n_rows != want) return 0;
        /* a tile's groups end before the next tile starts (the upload copies
         * byte ranges of whole tiles) */
        const uint64_t end = t + 1 < d->n_tiles ? d->tile_offsets[t + 1] : total;
        if (end <= o || o + 16 + (uint64_t)((th.n_rows + 7) / 8) * grp > end) return 0;
    }
    return 1;
}

static void set_devw(DpufDevW* out, const Upload* u, const DpufWeightDesc* d) {
    out->g = (const uint8_t*)u->d_groups;
    out->sign = (const uint8_t*)u->d_sign;
    out->rows = d->rows;
    out->cols = d->cols;
    out->n_groups = (d->rows + 7) / 8;
    out->mode = d->mode;
}

/* Weight upload at create: the .dpuf tile bytes go through two pinned host
 * buffers of UP_CHUNK bytes.  For each chunk of whole tiles the host copies
 * the bytes out of the caller's (typically mmapped) tensor into one pinned
 * buffer -- the page-in happens here -- while the DMA engine moves the other
 * buffer's previous chunk to HBM and k_relayout writes its tiles into the
 * row-block layout.  A buffer is refilled only after the event recorded
 * behind its last relayout has fired, and create synchronises once at the
 * end. */
#define UP_CHUNK ((size_t)16 << 20)

typedef struct {
    void* pin[2];        /* pinned host: tile bytes */
    uint64_t* pin_offs[2];
    void* dev[2];        /* device: the same chunk, relayout input */
    uint64_t* dev_offs[2];
    void* ev[2];
    int used[2];
    int next;
    int32_t max_tiles;   /* capacity of the offset tables */
} Stager;

static void stager_free(Stager* st) {
    for (int b = 0; b < 2; b++) {
        dpuf_hip_host_free(st->pin[b]);
        dpuf_hip_host_free(st->pin_offs[b]);
        dpuf_hip_free(st->dev[b]);
        dpuf_hip_free(st->dev_offs[b]);
        if (st->ev[b]) dpuf_hip_event_destroy(st->ev[b]);
    }
    memset(st, 0, sizeof *st);
}

static int stager_init(Stager* st) {
    memset(st, 0, sizeof *st);
    /* a chunk holds at least one tile: 16 + 2 * (16384 / 32) * 208 bytes at the
     * widest matrix create accepts, far below UP_CHUNK */
    st->max_tiles = (int32_t)(UP_CHUNK / 16) + 1;
    for (int b = 0; b < 2; b++) {
        st->pin[b] = dpuf_hip_host_alloc(UP_CHUNK);
        st->pin_offs[b] = (uint64_t*)dpuf_hip_host_alloc((size_t)st->max_tiles * 8u);
        st->dev[b] = dpuf_hip_malloc(UP_CHUNK);
        st->dev_offs[b] = (uint64_t*)dpuf_hip_malloc((size_t)st->max_tiles * 8u);
        st->ev[b] = dpuf_hip_event_create();
        if (!st->pin[b] || !st->pin_offs[b] || !st->dev[b] || !st->dev_offs[b] || !st->ev[b]) {
            stager_free(st);
            return 0;
        }
    }
    return 1;
}

/* Uploads tiles of d chunk by chunk into the row-block layout at dst. */
static void stage_tiles(Engine* e, Stager* st, const DpufWeightDesc* d, uint8_t* dst) {
    const int32_t n_blk = d->cols / 32;
    const uint64_t gbytes = (uint64_t)n_blk * (uint64_t)dpuf_grp_unit(d->mode);
    int32_t t0 = 0;
    while (t0 < d->n_tiles) {
        const uint64_t lo = d->tile_offsets[t0];
        int32_t t1 = t0 + 1;
        while (t1 < d->n_tiles && d->tile_offsets[t1 + 1] - lo <= UP_CHUNK && t1 - t0 + 1 < st->max_tiles) t1++;
        const uint64_t hi = d->tile_offsets[t1];
        const int b = st->next;
        st->next ^= 1;
        if (st->used[b]) dpuf_hip_event_sync(st->ev[b]);
        memcpy(st->pin[b], d->tensor_base + lo, (size_t)(hi - lo));
        for (int32_t t = t0; t <= t1; t++) st->pin_offs[b][t - t0] = d->tile_offsets[t] - lo;
        const int32_t r1 = 16 * t1 < d->rows ? 16 * t1 : d->rows;
        const int32_t n_groups = (r1 - 16 * t0 + 7) / 8;
        dpuf_hip_h2d(st->dev[b], st->pin[b], (size_t)(hi - lo), e->stream);
        dpuf_hip_h2d(st->dev_offs[b], st->pin_offs[b], (size_t)(t1 - t0 + 1) * 8u, e->stream);
        dpuf_hip_relayout(e->stream, (const uint8_t*)st->dev[b], st->dev_offs[b], n_groups, n_blk, d->mode,
                          dst + (size_t)(2 * t0) * gbytes);
        dpuf_hip_event_record(st->ev[b], e->stream);
        st->used[b] = 1;
        t0 = t1;
    }
}

/* Uploads one validated mode 12 / 13 / 14 matrix (tied tensors once). */
static int upload_desc(Engine* e, Stager* st, const DpufWeightDesc* d, DpufDevW* out) {
    if (!validate_desc(d)) return 0;
    for (int32_t i = 0; i < e->n_ups; i++) {
        if (e->ups[i].host_base == d->tensor_base) {
            set_devw(out, &e->ups[i], d);
            return 1;
        }
    }
    Upload u;
    memset(&u, 0, sizeof u);
    u.host_base = d->tensor_base;
    const int32_t n_groups = (d->rows + 7) / 8, n_blk = d->cols / 32;
    u.bytes = (uint64_t)n_groups * (uint64_t)n_blk * (uint64_t)dpuf_grp_unit(d->mode);
    u.d_groups = dpuf_hip_malloc((size_t)u.bytes);
    if (d->sign_bits) u.d_sign = dpuf_hip_malloc((size_t)d->cols / 8u);
    if (!u.d_groups || (d->sign_bits && !u.d_sign)) {
        dpuf_hip_free(u.d_groups); dpuf_hip_free(u.d_sign);
        return 0;
    }
    Upload* grown = (Upload*)realloc(e->ups, (size_t)(e->n_ups + 1) * sizeof(Upload));
    if (!grown) {
        dpuf_hip_free(u.d_groups); dpuf_hip_free(u.d_sign);
        return 0;
    }
    e->ups = grown;
    e->ups[e->n_ups++] = u;  /* owned by the engine from here on, also on failure */
    if (d->sign_bits) dpuf_hip_h2d(u.d_sign, d->sign_bits, (size_t)d->cols / 8u, e->stream);
    stage_tiles(e, st, d, (uint8_t*)u.d_groups);
    set_devw(out, &u, d);
    return dpuf_hip_ok();
}

static float* upload_floats(Engine* e, const float* src, size_t n) {
    if (!src) return NULL;
    float* d = (float*)dpuf_hip_malloc(n * sizeof(float));
    if (!d) return NULL;
    dpuf_hip_h2d(d, src, n * sizeof(float), e->stream);
    return d;
}

static int same_signs(const DpufWeightDesc* a, const DpufWeightDesc* b) {
    if (a->cols != b->cols) return 0;
    if (!a->sign_bits || !b->sign_bits) return a->sign_bits == b->sign_bits;
    return memcmp(a->sign_bits, b->sign_bits, (size_t)a->cols / 8u) == 0;
}

/* RoPE tables on the host with the C library, exactly as the reference's
 * precompute_rope (dpuf_engine.c:183-223), then uploaded. */
static int rope_tables(Engine* e) {
    const int32_t half = e->hd >> 1;
    const DpufModelConfig* c = &e->cfg;
    float* inv_freq = (float*)malloc((size_t)half * sizeof(float));
    float* ct = (float*)malloc((size_t)e->max_seq * half * sizeof(float));
    float* st = (float*)malloc((size_t)e->max_seq * half * sizeof(float));
    if (!inv_freq || !ct || !st) { free(inv_freq); free(ct); free(st); return 0; }
    for (int32_t j = 0; j < half; j++) {
        float freq = 1.0f / powf(c->rope_theta, (float)(2 * j) / (float)e->hd);
        if (c->use_llama3_rope) {
            float factor = c->rope_factor, low_f = c->rope_low_freq, high_f = c->rope_high_freq;
            float orig_max = (float)c->rope_orig_max_pos;
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
    for (int32_t p = 0; p < e->max_seq; p++)
        for (int32_t j = 0; j < half; j++) {
            float ang = (float)p * inv_freq[j];
            ct[(size_t)p * half + j] = cosf(ang);
            st[(size_t)p * half + j] = sinf(ang);
        }
    e->d_cos = upload_floats(e, ct, (size_t)e->max_seq * half);
    e->d_sin = upload_floats(e, st, (size_t)e->max_seq * half);
    int ok = e->d_cos && e->d_sin && dpuf_hip_sync(e->stream) == 0;
    free(inv_freq); free(ct); free(st);
    return ok;
}

static int is_q8(const Engine* e) { return e->cfg.kv_type == DPUF_KV_Q8; }

static void kv_layout(Engine* e) {
    const size_t hd = (size_t)e->hd;
    if (is_q8(e)) {
        e->kv_n = 4;
        e->kv_row[0] = e->kv_row[1] = hd;
        e->kv_row[2] = e->kv_row[3] = (hd / 32) * sizeof(float);
    } else {
        e->kv_n = 2;
        e->kv_row[0] = e->kv_row[1] = hd * sizeof(float);
    }
}

/* Bytes of KV array i for `len` positions of every (layer, kv head). */
static size_t kv_bytes(const Engine* e, int i, int32_t len) {
    return (size_t)e->L * (size_t)e->nkv * (size_t)len * e->kv_row[i];
}

static float* slot_k(const Engine* e, int32_t s) { return (float*)e->kv[s][0]; }
static float* slot_v(const Engine* e, int32_t s) { return (float*)e->kv[s][1]; }

/* The int8 cache of layer l of slot s. */
static DpufKvQ8 slot_q8(const Engine* e, int32_t s, int32_t l) {
    const size_t rows = (size_t)l * e->nkv * e->max_seq;
    DpufKvQ8 c;
    c.kq = (int8_t*)e->kv[s][0] + rows * e->kv_row[0];
    c.vq = (int8_t*)e->kv[s][1] + rows * e->kv_row[1];
    c.ks = (float*)((uint8_t*)e->kv[s][2] + rows * e->kv_row[2]);
    c.vs = (float*)((uint8_t*)e->kv[s][3] + rows * e->kv_row[3]);
    return c;
}

static void kv_free(void* a[4]) {
    for (int i = 0; i < 4; i++) {
        dpuf_hip_free(a[i]);
        a[i] = NULL;
    }
}

static int slot_alloc(Engine* e, int32_t s) {
    if (e->kv[s][0]) return 1;
    for (int i = 0; i < e->kv_n; i++) {
        e->kv[s][i] = dpuf_hip_malloc(kv_bytes(e, i, e->max_seq));
        if (!e->kv[s][i]) {
            kv_free(e->kv[s]);
            return 0;
        }
        dpuf_hip_fill_zero(e->kv[s][i], kv_bytes(e, i, e->max_seq), e->stream);
    }
    return dpuf_hip_sync(e->stream) == 0;
}

/* Positions [0, len) of every (layer, kv head) between a slot ([..][max_seq]
 * rows) and a prefix ([..][len] rows), to_prefix selecting the direction. */
static void prefix_copy(Engine* e, int32_t s, int32_t p, int32_t len, int to_prefix) {
    for (int i = 0; i < e->kv_n; i++) {
        const size_t rb = e->kv_row[i];
        for (int32_t lh = 0; lh < e->L * e->nkv; lh++) {
            uint8_t* so = (uint8_t*)e->kv[s][i] + (size_t)lh * e->max_seq * rb;
            uint8_t* po = (uint8_t*)e->pkv[p][i] + (size_t)lh * len * rb;
            if (to_prefix) dpuf_hip_d2d(po, so, (size_t)len * rb, e->stream);
            else dpuf_hip_d2d(so, po, (size_t)len * rb, e->stream);
        }
    }
}

static void engine_free(Engine* e) {
    if (!e) return;
    dpuf_hip_bind_error_word(NULL);
    if (e->stream) dpuf_hip_sync(e->stream);
    for (int i = 0; i < N_GRAPHS; i++) dpuf_hip_graph_destroy(e->graphs[i]);
    for (int32_t i = 0; i < e->n_ups; i++) {
        dpuf_hip_free(e->ups[i].d_groups); dpuf_hip_free(e->ups[i].d_sign);
    }
    free(e->ups);
    if (e->d_norm) {
        for (int32_t i = 0; i < 4 * e->L; i++) dpuf_hip_free(e->d_norm[i]);
        free(e->d_norm);
    }
    free(e->lw);
    free(e->q_idx);
    dpuf_hip_free(e->d_out_norm); dpuf_hip_free(e->d_cos); dpuf_hip_free(e->d_sin);
    for (int s = 0; s < N_SLOTS; s++) kv_free(e->kv[s]);
    for (int p = 0; p < N_PREFIX; p++) kv_free(e->pkv[p]);
    float* bufs[] = {e->h, e->h2, e->hn, e->q, e->k, e->v, e->ao, e->gate, e->up, e->logits, e->scores, e->embeds,
                     e->capture};
    for (size_t i = 0; i < sizeof bufs / sizeof bufs[0]; i++) dpuf_hip_free(bufs[i]);
    for (int i = 0; i < 3; i++) {
        dpuf_hip_free(e->prep[i].q);
        dpuf_hip_free(e->prep[i].s);
        dpuf_hip_free(e->prep[i].m);
        dpuf_hip_free(e->prep[i].h);
    }
    dpuf_hip_free(e->d_ids);
    dpuf_hip_free(e->d_pflag);
    dpuf_hip_free(e->d_red);
    dpuf_hip_free(e->d_lmred);
    dpuf_hip_free(e->d_ms_kc);
    dpuf_hip_host_free(e->h_pinned);
    dpuf_hip_host_free(e->h_io);
    dpuf_hip_host_free(e->h_logits);
    dpuf_hip_host_free(e->h_emb);
    dpuf_hip_host_free(e->h_ms);
    dpuf_hip_host_free(e->h_tok);
    for (int i = 0; i < MAX_EVENTS; i++) if (e->ev[i]) dpuf_hip_event_destroy(e->ev[i]);
    if (e->stream) dpuf_hip_stream_destroy(e->stream);
    free(e);
}

DPUF_EXPORT int32_t dpuf_amd_device_ok(void) { return dpuf_hip_device_count() > 0; }
DPUF_EXPORT const char* dpuf_amd_last_error(void) { return dpuf_hip_error_string(); }

DPUF_EXPORT void* dpuf_engine_create(const DpufModelConfig* cfg, const DpufLayerWeights* layers,
                                     const DpufWeightDesc* w_tok_embd, const DpufWeightDesc* w_lm_head,
                                     const float* output_norm) {
    dpuf_hip_clear_error();
    if (!cfg || !layers || !w_tok_embd || !w_lm_head || !output_norm) return NULL;
    /* head dims 64, 128, 256 and groups of at most 32 query heads per KV head:
     * the shapes the attention kernels are built and tested for */
    if (cfg->num_layers < 0 || cfg->hidden_size <= 0 ||
        (cfg->head_dim != 64 && cfg->head_dim != 128 && cfg->head_dim != 256) || cfg->num_kv_heads <= 0 ||
        cfg->num_q_heads <= 0 || (cfg->num_q_heads % cfg->num_kv_heads) != 0 ||
        cfg->num_q_heads / cfg->num_kv_heads > 32 || cfg->max_seq_len <= 0 || cfg->vocab_size <= 0 ||
        (cfg->kv_type != DPUF_KV_F32 && cfg->kv_type != DPUF_KV_Q8) || cfg->has_mrope || (cfg->hidden_size % 64) != 0 ||
        cfg->hidden_size < 128 || cfg->hidden_size > 16384 ||
        (cfg->intermediate_size % 64) != 0)
        return NULL;
    if (dpuf_hip_device_count() <= 0) return NULL;
    Engine* e = (Engine*)calloc(1, sizeof(Engine));
    if (!e) return NULL;
    Stager stg;
    memset(&stg, 0, sizeof stg);
    e->cfg = *cfg;
    e->L = cfg->num_layers;
    e->H = cfg->hidden_size;
    e->I = cfg->intermediate_size;
    e->nq = cfg->num_q_heads;
    e->nkv = cfg->num_kv_heads;
    e->hd = cfg->head_dim;
    e->qd = e->nq * e->hd;
    e->kvd = e->nkv * e->hd;
    e->V = cfg->vocab_size;
    e->max_seq = cfg->max_seq_len;
    kv_layout(e);
    const char* dz = getenv("DPUF_SWIGLU_DEADZONE");
    e->deadzone = dz ? (float)atof(dz) : 0.005f;
    e->stream = dpuf_hip_stream_create();
    if (!e->stream) goto fail;

    /* weights: descriptors must match the config's shapes */
    e->lw = (DpufDevW*)calloc((size_t)(e->L > 0 ? e->L : 1) * 7u, sizeof(DpufDevW));
    e->d_norm = (float**)calloc((size_t)(e->L > 0 ? e->L : 1) * 4u, sizeof(float*));
    e->q_idx = (uint8_t*)calloc((size_t)(e->L > 0 ? e->L : 1) * 5u, 1);
    if (!e->lw || !e->d_norm || !e->q_idx) goto fail;
    if (w_tok_embd->rows != e->V || w_tok_embd->cols != e->H || w_lm_head->rows != e->V || w_lm_head->cols != e->H)
        goto fail;
    if (!stager_init(&stg)) goto fail;
    if (!upload_desc(e, &stg, w_tok_embd, &e->tok) || !upload_desc(e, &stg, w_lm_head, &e->lm)) goto fail;
    for (int32_t l = 0; l < e->L; l++) {
        const DpufLayerWeights* lw = &layers[l];
        const DpufWeightDesc* ds[7] = {&lw->w_q, &lw->w_k, &lw->w_v, &lw->w_o, &lw->w_gate, &lw->w_up, &lw->w_down};
        const int32_t want_r[7] = {e->qd, e->kvd, e->kvd, e->H, e->I, e->I, e->H};
        const int32_t want_c[7] = {e->H, e->H, e->H, e->qd, e->H, e->H, e->I};
        for (int k = 0; k < 7; k++) {
            if (ds[k]->rows != want_r[k] || ds[k]->cols != want_c[k]) goto fail;
            if (!upload_desc(e, &stg, ds[k], &e->lw[(size_t)l * 7 + k])) goto fail;
        }
        if (!lw->attn_norm || !lw->ffn_norm) goto fail;
        e->d_norm[4 * l + 0] = upload_floats(e, lw->attn_norm, (size_t)e->H);
        if (cfg->has_qk_norm && lw->attn_q_norm) e->d_norm[4 * l + 1] = upload_floats(e, lw->attn_q_norm, (size_t)e->hd);
        if (cfg->has_qk_norm && lw->attn_k_norm) e->d_norm[4 * l + 2] = upload_floats(e, lw->attn_k_norm, (size_t)e->hd);
        e->d_norm[4 * l + 3] = upload_floats(e, lw->ffn_norm, (size_t)e->H);
        if (!e->d_norm[4 * l + 0] || !e->d_norm[4 * l + 3]) goto fail;
        /* shared activation prep when sign vectors agree (dpuf_engine.c:887-897) */
        /* qi[0..2]: prep index of Q, K, V; qi[3]: distinct preps; qi[4]: up's */
        uint8_t* qi = e->q_idx + 5 * (size_t)l;
        const DpufWeightDesc* qkv[3] = {&lw->w_q, &lw->w_k, &lw->w_v};
        int rep[3], n = 0;
        for (int k = 0; k < 3; k++) {
            int found = -1;
            for (int j = 0; j < n && found < 0; j++)
                if (same_signs(qkv[rep[j]], qkv[k])) found = j;
            if (found < 0) { rep[n] = k; found = n++; }
            qi[k] = (uint8_t)found;
        }
        qi[3] = (uint8_t)n;
        qi[4] = same_signs(&lw->w_gate, &lw->w_up) ? 0 : 1;
    }
    e->d_out_norm = upload_floats(e, output_norm, (size_t)e->H);
    if (!e->d_out_norm || !rope_tables(e)) goto fail;
    for (int32_t i = 0; i < e->n_ups; i++) e->weight_bytes += e->ups[i].bytes;

    /* scratch */
    {
        const size_t B = DPUF_AMD_MAX_BATCH;
        int32_t maxd = e->H > e->I ? e->H : e->I;
        if (e->qd > maxd) maxd = e->qd;
        e->h = (float*)dpuf_hip_malloc(B * e->H * 4);
        e->h2 = (float*)dpuf_hip_malloc(B * e->H * 4);
        e->hn = (float*)dpuf_hip_malloc(B * e->H * 4);
        e->q = (float*)dpuf_hip_malloc(B * e->qd * 4);
        e->k = (float*)dpuf_hip_malloc(B * e->kvd * 4);
        e->v = (float*)dpuf_hip_malloc(B * e->kvd * 4);
        e->ao = (float*)dpuf_hip_malloc(B * e->qd * 4);
        e->gate = (float*)dpuf_hip_malloc(B * e->I * 4);
        e->up = (float*)dpuf_hip_malloc(B * e->I * 4);
        e->logits = (float*)dpuf_hip_malloc(B * (size_t)e->V * 4);
        e->scores = (float*)dpuf_hip_malloc(B * (size_t)e->nq * e->max_seq * 4);
        e->embeds = (float*)dpuf_hip_malloc(B * e->H * 4);
        for (int i = 0; i < 3; i++) {
            e->prep[i].q = (int8_t*)dpuf_hip_malloc(B * maxd);
            e->prep[i].s = (float*)dpuf_hip_malloc(B * (maxd / 32) * 4);
            e->prep[i].m = (int32_t*)dpuf_hip_malloc(B * (maxd / 32) * 4);
            e->prep[i].h = (uint16_t*)dpuf_hip_malloc(B * maxd * 2);
            if (!e->prep[i].q || !e->prep[i].s || !e->prep[i].m || !e->prep[i].h) goto fail;
        }
        e->d_ids = (int32_t*)dpuf_hip_malloc((B + 64) * 4);
        e->h_pinned = (int32_t*)dpuf_hip_host_alloc((B + 64) * 4);
        e->h_io = (int32_t*)dpuf_hip_host_alloc_io((B + 64) * 4);
        e->h_logits = (float*)dpuf_hip_host_alloc_io((size_t)e->V * 4);
        e->h_emb = (float*)dpuf_hip_host_alloc_io((size_t)e->H * 4);
        e->h_ms = dpuf_hip_host_alloc(B * 2 * sizeof(float*) + B * 4);
        e->h_tok = (int32_t*)dpuf_hip_host_alloc_io(B * 4);
        e->d_red = dpuf_hip_malloc(DPUF_HIP_RED_SCRATCH);
        e->d_lmred = dpuf_hip_malloc((size_t)(LM_RED_CAP + 1) * 16);
        e->d_ms_kc = (float**)dpuf_hip_malloc(B * 2 * sizeof(float*) + B * 8);
        if (!e->d_ms_kc) goto fail;
        e->d_ms_vc = e->d_ms_kc + B;
        e->d_ms_pos = (int32_t*)(e->d_ms_vc + B);
        e->d_ms_tok = e->d_ms_pos + B;
        if (!e->h || !e->h2 || !e->hn || !e->q || !e->k || !e->v || !e->ao || !e->gate || !e->up || !e->logits ||
            !e->scores || !e->embeds || !e->d_ids || !e->h_pinned || !e->h_io || !e->h_logits || !e->h_emb || !e->d_red || !e->d_lmred || !e->h_ms || !e->h_tok)
            goto fail;
        e->d_pos0 = e->d_ids + B;
        e->d_flag = e->d_ids + B + 1;
        e->d_tok = e->d_ids + B + 2;
        e->d_err = e->d_ids + B + 3;
        e->d_serial = e->d_ids + B + 4;
        e->d_pflag = (int32_t*)dpuf_hip_malloc((size_t)(e->L > 0 ? e->L : 1) * 1024 * 4);
        if (!e->d_pflag) goto fail;
        dpuf_hip_fill_zero(e->d_pflag, (size_t)(e->L > 0 ? e->L : 1) * 1024 * 4, e->stream);
        dpuf_hip_fill_zero(e->d_ids, (B + 64) * 4, e->stream);
        memset(e->h_io, 0, (B + 64) * 4);
        dpuf_hip_fill_zero(e->hn, B * e->H * 4, e->stream);
    }
    if (!slot_alloc(e, 0)) goto fail;
    if (dpuf_hip_sync(e->stream) != 0) goto fail;
    stager_free(&stg);
    return e;
fail:
    if (e->stream) dpuf_hip_sync(e->stream);
    stager_free(&stg);
    engine_free(e);
    return NULL;
}

DPUF_EXPORT void dpuf_engine_destroy(void* handle) { engine_free((Engine*)handle); }

DPUF_EXPORT int32_t dpuf_engine_set_slot(void* handle, int32_t slot_id) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || slot_id < 0 || slot_id >= N_SLOTS) return -1;
    if (!slot_alloc(e, slot_id)) return -2;
    e->active = slot_id;
    return 0;
}

DPUF_EXPORT int32_t dpuf_engine_get_slot(void* handle) {
    Engine* e = (Engine*)handle;
    return e ? e->active : 0;
}

DPUF_EXPORT int32_t dpuf_engine_num_slots(void* handle) { return handle ? N_SLOTS : 1; }

DPUF_EXPORT void dpuf_engine_reset_slot(void* handle, int32_t slot_id) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || slot_id < 0 || slot_id >= N_SLOTS || !e->kv[slot_id][0]) return;
    for (int i = 0; i < e->kv_n; i++) dpuf_hip_fill_zero(e->kv[slot_id][i], kv_bytes(e, i, e->max_seq), e->stream);
    dpuf_hip_sync(e->stream);
}

DPUF_EXPORT void dpuf_engine_reset_cache(void* handle) {
    Engine* e = (Engine*)handle;
    if (!e) return;
    dpuf_engine_reset_slot(handle, e->active);
}

DPUF_EXPORT size_t dpuf_engine_slot_memory(void* handle) {
    Engine* e = (Engine*)handle;
    if (!e) return 0;
    size_t n = 0;
    for (int i = 0; i < e->kv_n; i++) n += kv_bytes(e, i, e->max_seq);
    return n;
}

/* Prefix caches are [L][kv head][len][hd] (dpuf_engine.c:1471-1600). */
DPUF_EXPORT int32_t dpuf_engine_freeze_prefix(void* handle, int32_t pfx_id, int32_t prefix_len) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || pfx_id < 0 || pfx_id >= N_PREFIX || prefix_len <= 0 || prefix_len > e->max_seq) return 0;
    /* a prefix's arrays hold exactly its length: [L][kv head][len] rows */
    if (e->pcap[pfx_id] != prefix_len || !e->pkv[pfx_id][0]) {
        kv_free(e->pkv[pfx_id]);
        e->pvalid[pfx_id] = 0;
        e->pcap[pfx_id] = 0;
        for (int i = 0; i < e->kv_n; i++) {
            e->pkv[pfx_id][i] = dpuf_hip_malloc(kv_bytes(e, i, prefix_len));
            if (!e->pkv[pfx_id][i]) {
                kv_free(e->pkv[pfx_id]);
                return 0;
            }
        }
        e->pcap[pfx_id] = prefix_len;
    }
    if (!e->kv[e->active][0]) return 0;
    prefix_copy(e, e->active, pfx_id, prefix_len, 1);
    if (dpuf_hip_sync(e->stream) != 0) return 0;
    e->plen[pfx_id] = prefix_len;
    e->pvalid[pfx_id] = 1;
    return 1;
}

DPUF_EXPORT int32_t dpuf_engine_apply_prefix(void* handle, int32_t slot_id, int32_t pfx_id) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || slot_id < 0 || slot_id >= N_SLOTS || pfx_id < 0 || pfx_id >= N_PREFIX) return 0;
    if (!e->pvalid[pfx_id] || e->plen[pfx_id] <= 0) return 0;
    if (!slot_alloc(e, slot_id)) return 0;
    const int32_t len = e->plen[pfx_id];
    prefix_copy(e, slot_id, pfx_id, len, 0);
    if (dpuf_hip_sync(e->stream) != 0) return 0;
    return len;
}

DPUF_EXPORT int32_t dpuf_engine_get_prefix_len(void* handle, int32_t pfx_id) {
    Engine* e = (Engine*)handle;
    if (!e || pfx_id < 0 || pfx_id >= N_PREFIX) return 0;
    return e->pvalid[pfx_id] ? e->plen[pfx_id] : 0;
}

/* ------------------------------------------------------------------------- */
/* Forward                                                                    */
/* ------------------------------------------------------------------------- */

/* Algorithmic bytes of one GEMV launch over tiles [t0, t1): the weight
 * groups (8 rows x 32 columns = 144 bytes each, 208 for mode 14) plus, per
 * token row, the prepped activations (K int8 + 8 bytes per 32-block) and the
 * fp32 outputs. */
static double gemv_bytes(const DpufDevW* w, int32_t t0, int32_t t1, int32_t M) {
    const int32_t g0 = 2 * t0, g1 = 2 * t1 < w->n_groups ? 2 * t1 : w->n_groups;
    const int32_t r1 = 16 * t1 < w->rows ? 16 * t1 : w->rows;
    const double n_blk = (double)(w->cols / 32);
    return (double)(g1 - g0) * n_blk * dpuf_grp_unit(w->mode) +
           (double)M * (w->cols + n_blk * 8.0 + (r1 - 16 * t0) * 4.0);
}

/* Tiles [t0, t1) of w (16 rows each) as a GEMV job over 8-row groups. */
static DpufGemvJob job(const DpufDevW* w, int32_t t0, int32_t t1, DpufPrep p, float* out, int32_t ldo) {
    DpufGemvJob j;
    j.w = *w;
    j.g0 = 2 * t0;
    j.g1 = 2 * t1 < w->n_groups ? 2 * t1 : w->n_groups;
    j.p = p;
    j.out = out;
    j.ldo = ldo;
    return j;
}

static int32_t n_tiles_of(const DpufDevW* w) { return (w->rows + 15) / 16; }


static void enqueue_layers(Engine* e, int32_t M, int32_t keep_tiles);
static int enqueue_head(Engine* e, int32_t M, int32_t only_last, int32_t early_tiles, float early_margin,
                        int32_t want_argmax, float* lm_host);

/* Whether the LM head of a step runs the Zone-A early exit (one row, the
 * vocabulary above 2048 tiles, zone tiles set). */
/* The serial of the next forward call: positive, never the same twice in a
 * row of 2^31 - 1 calls, never 0 (the producer flags start at 0). */
static int32_t next_serial(Engine* e) {
    e->serial = e->serial >= 0x7FFFFFFF - 1 ? 1 : e->serial + 1;
    return e->serial;
}

static int head_early(const Engine* e, int32_t lm_rows, int32_t early_tiles) {
    return early_tiles > 0 && lm_rows == 1 && n_tiles_of(&e->lm) > 2048;
}

/* Enqueues one forward step: ids in h_io[0, M) and pos0 in h_io[IO_POS];
 * rows with id -1 take their hidden state from h_emb (M == 1: every one-row
 * step, graphs included, points the embedding kernel there, and a row with a
 * token id ignores it) or, for M > 1 with use_embeds, from e->embeds on the
 * device.  lm_host, when set, takes the one LM-head row in place of
 * e->logits.  Ends by publishing the flag, token and error word to
 * h_io[IO_OUT..]. */
static void enqueue_forward(Engine* e, int32_t M, int32_t use_embeds, int32_t only_last, int32_t keep_tiles,
                            int32_t early_tiles, float early_margin, int32_t want_argmax, float* lm_host) {
    const float* emb = M == 1 ? e->h_emb : use_embeds ? e->embeds : NULL;
    dpuf_hip_embed(e->stream, e->tok, e->h_io, M, emb, M == 1, e->h, e->h_io + IO_POS, e->d_pos0, e->d_serial);
    e->hcur = e->h;
    enqueue_layers(e, M, keep_tiles);
    const int hr = enqueue_head(e, M, only_last, early_tiles, early_margin, want_argmax, lm_host);
    if (!(hr & 2)) dpuf_hip_publish(e->stream, e->d_flag, hr & 1, e->h_io + IO_OUT);
}

/* Layer loop: residual + RMSNorm + prep, fused Q/K/V GEMV, attention (for
 * M == 1 one kernel with QK-norm, RoPE, the KV store and the O-input prep),
 * O GEMV, residual + RMSNorm + prep, fused gate/up GEMV, SwiGLU + prep, down
 * GEMV; the residual stream is e->hcur (e->h or e->h2) and the last projection
 * e->hn. */
static float* h_other(const Engine* e) { return e->hcur == e->h ? e->h2 : e->h; }

/* The one-row GEMV jobs of layer l: Q/K/V, O, gate/up, down (pruned to
 * keep_tiles). */
typedef struct {
    DpufGemvJob qkv[3], o, gu[2], down;
} LayerJobs;

static LayerJobs layer_jobs(Engine* e, int32_t l, int32_t keep_tiles) {
    const DpufDevW* W = e->lw + (size_t)l * 7;
    const uint8_t* qi = e->q_idx + (size_t)l * 5;
    LayerJobs r;
    r.qkv[0] = job(&W[W_Q], 0, n_tiles_of(&W[W_Q]), e->prep[qi[0]], e->q, e->qd);
    r.qkv[1] = job(&W[W_K], 0, n_tiles_of(&W[W_K]), e->prep[qi[1]], e->k, e->kvd);
    r.qkv[2] = job(&W[W_V], 0, n_tiles_of(&W[W_V]), e->prep[qi[2]], e->v, e->kvd);
    r.o = job(&W[W_O], 0, n_tiles_of(&W[W_O]), e->prep[0], e->hn, e->H);
    r.gu[0] = job(&W[W_GATE], 0, n_tiles_of(&W[W_GATE]), e->prep[0], e->gate, e->I);
    r.gu[1] = job(&W[W_UP], 0, n_tiles_of(&W[W_UP]), e->prep[qi[4]], e->up, e->I);
    const int32_t nt = n_tiles_of(&W[W_DOWN]);
    const int32_t kt = (keep_tiles > 0 && keep_tiles < nt) ? keep_tiles : nt;
    r.down = job(&W[W_DOWN], 0, kt, e->prep[0], e->hn, e->H);
    return r;
}

/* What the decode attention of layer l warms while its workgroups run on a
 * few CUs: the O projection after it, the first round of gate/up, and the
 * next layer's Q/K/V (the Infinity Cache keeps them across the launches in
 * between).  The down projection and the later gate/up rounds stay cold:
 * reading them too made the attention launch longer than the GEMVs gained. */
static DpufWarm attn_warm(Engine* e, const LayerJobs* lj, const LayerJobs* ln) {
    DpufWarm w;
    memset(&w, 0, sizeof w);
    dpuf_hip_warm_add(&w, 1, &lj->o, 0, 1);
    dpuf_hip_warm_add(&w, 2, lj->gu, 0, 1);
    if (ln) dpuf_hip_warm_add(&w, 3, ln->qkv, 0, 1);
    w.sink = e->d_ids + DPUF_AMD_MAX_BATCH + 8;
    return w;
}

/* What the P.V launch of a long-context one-token step warms on the CUs its
 * chain workgroups leave idle (about 17 us at 4 096 keys): the same groups,
 * with the O groups on the XCDs of the workgroups that read them (that O
 * launch preps its own input in producer workgroups ahead of its GEMV
 * workgroups), and two gate/up rounds instead of one.  Measured at 4 096
 * keys: one gate/up round 3.14 -> 3.08 ms/token, two 3.05, three 3.19, four
 * 3.32 (the P.V launch then outlasts its chains); the down projection as
 * well, 3.84. */
static DpufWarm attn_warm_fed_o(Engine* e, const LayerJobs* lj, const LayerJobs* ln) {
    DpufWarm w;
    memset(&w, 0, sizeof w);
    if (dpuf_hip_warm_add(&w, 1, &lj->o, 0, 1)) w.j[0].wb += dpuf_hip_fed_producers(e->qd, &lj->o);
    dpuf_hip_warm_add(&w, 2, lj->gu, 0, 2);
    if (ln) dpuf_hip_warm_add(&w, 3, ln->qkv, 0, 1);
    w.sink = e->d_ids + DPUF_AMD_MAX_BATCH + 8;
    return w;
}

/* Attention of a multi-session step at layer l (ms_n = M tokens, one per
 * session): the first ms_short tokens (fp32 cache, short context) in one
 * fused decode launch over their sessions' caches; every other token alone,
 * at its own position against its own slot's cache, through the one-token
 * kernels a single-session step of that length takes (dpuf_engine.c:1404-1600
 * serves each slot's sequence the same way); then, when any token took the
 * latter, the O-input prep of all M rows (the fused kernel's rows prep to the
 * same values). */
static void enqueue_ms_attention(Engine* e, int32_t l, int32_t M, float eps, float scale, const uint8_t* o_sign) {
    void* s = e->stream;
    const DpufWarm no_warm = {0};
    const size_t lo = (size_t)l * e->nkv * e->max_seq * e->hd;
    const int32_t ns = e->ms_short;
    const float *qn = e->d_norm[4 * l + 1], *kn = e->d_norm[4 * l + 2];
    if (ns > 0)
        dpuf_hip_attn_dec(s, ns, e->q, e->k, e->v, qn, kn, eps, e->d_cos, e->d_sin, NULL, NULL, e->d_ms_pos, e->nq,
                          e->nkv, e->hd, e->max_seq, scale, e->ao, o_sign, e->prep[0], e->d_ms_kc, e->d_ms_vc, lo,
                          no_warm);
    for (int32_t m = ns; m < M; m++) {
        float* q = e->q + (size_t)m * e->qd;
        float* k = e->k + (size_t)m * e->kvd;
        float* v = e->v + (size_t)m * e->kvd;
        float* ao = e->ao + (size_t)m * e->qd;
        const int32_t* pp = e->d_ms_pos + m;
        const int32_t keys = e->ms_pos[m] + 1;
        if (is_q8(e)) {
            const DpufKvQ8 c8 = slot_q8(e, e->ms_slot[m], l);
            dpuf_hip_qk_rope_kv(s, 1, q, k, v, qn, kn, eps, e->d_cos, e->d_sin, NULL, NULL, pp, e->nq, e->nkv, e->hd,
                                e->max_seq, &c8);
            dpuf_hip_attn_q8(s, 1, keys, q, c8, ao, e->scores, pp, e->nq, e->nkv, e->hd, e->max_seq, scale, NULL);
            continue;
        }
        float* kc = slot_k(e, e->ms_slot[m]) + lo;
        float* vc = slot_v(e, e->ms_slot[m]) + lo;
        if (dpuf_hip_attn_decode_rope(s, keys, q, k, v, qn, kn, eps, e->d_cos, e->d_sin, kc, vc, ao, e->scores, pp,
                                      e->nq, e->nkv, e->hd, e->max_seq, scale, NULL) == 0)
            continue;
        dpuf_hip_qk_rope_kv(s, 1, q, k, v, qn, kn, eps, e->d_cos, e->d_sin, kc, vc, pp, e->nq, e->nkv, e->hd,
                            e->max_seq, NULL);
        DpufPrep none;
        memset(&none, 0, sizeof none);
        if (dpuf_hip_attn_split(s, 1, keys, q, kc, vc, ao, e->scores, pp, e->nq, e->nkv, e->hd, e->max_seq, scale,
                                NULL, none, NULL) != 0)
            dpuf_hip_attn(s, 1, q, kc, vc, ao, e->scores, pp, e->nq, e->nkv, e->hd, e->max_seq, scale);
    }
    if (ns < M) dpuf_hip_prep(s, M, e->qd, e->ao, o_sign, e->prep[0]);
}

static void enqueue_layers(Engine* e, int32_t M, int32_t keep_tiles) {
    void* s = e->stream;
    const int32_t H = e->H, I = e->I;
    const float eps = e->cfg.rms_eps;
    const float scale = 1.0f / sqrtf((float)e->hd);
    for (int32_t l = 0; l < e->L; l++) {
        const DpufDevW* W = e->lw + (size_t)l * 7;
        const uint8_t* qi = e->q_idx + (size_t)l * 5;
        const size_t lo = (size_t)l * e->nkv * e->max_seq * e->hd;
        float* kc = is_q8(e) ? NULL : slot_k(e, e->active) + lo;
        float* vc = is_q8(e) ? NULL : slot_v(e, e->active) + lo;
        /* the layer's GEMV jobs (and the next layer's, whose Q/K/V the
         * decode attention warms) */
        const LayerJobs lj = layer_jobs(e, l, keep_tiles);
        LayerJobs ln_;
        const LayerJobs* ln = NULL;
        if (l + 1 < e->L) {
            ln_ = layer_jobs(e, l + 1, keep_tiles);
            ln = &ln_;
        }
        const DpufGemvJob* jqkv = lj.qkv;
        const DpufGemvJob jo = lj.o;
        const DpufGemvJob* jgu = lj.gu;
        int o_prep = 0; /* the O input still needs its prep (one-row steps) */

        /* (1) [h += down] + attn RMSNorm + prep of the Q/K/V input */
        {
            const uint8_t* signs[3] = {W[W_Q].sign, W[W_K].sign, W[W_V].sign};
            const int32_t np = qi[3];
            const uint8_t* ps[3] = {NULL, NULL, NULL};
            for (int k = 2; k >= 0; k--) ps[qi[k]] = signs[k];
            const int tm1 = tm_begin(e, K_PREP, 0);
            float* ho = l > 0 ? h_other(e) : NULL;
            dpuf_hip_resnorm_prep(s, M, H, e->hcur, l > 0 ? e->hn : NULL, ho, e->d_norm[4 * l], eps, np, ps, e->prep,
                                  NULL);
            if (ho) e->hcur = ho;
            tm_end(e, tm1);
        }
        /* (2) Q, K, V in one launch */
        {
            const DpufGemvJob* js = jqkv;
            double b = gemv_bytes(&W[W_Q], 0, n_tiles_of(&W[W_Q]), M) + gemv_bytes(&W[W_K], 0, n_tiles_of(&W[W_K]), M) +
                       gemv_bytes(&W[W_V], 0, n_tiles_of(&W[W_V]), M);
            const int tm2 = tm_begin(e, K_QKV, b);
            dpuf_hip_gemv(s, M, 3, js, NULL, 0.0f);
            tm_end(e, tm2);
        }
        /* (3) QK-norm + RoPE + KV store, (4) attention, (5) prep of the O input */
        {
            const int tm = tm_begin(e, K_ATTN, 0);
            int fused = 0;
            if (e->ms_n > 0) {
                /* one token per session, each against its own slot's cache */
                enqueue_ms_attention(e, l, M, eps, scale, W[W_O].sign);
                fused = 1;
            } else if (is_q8(e)) {
                /* int8 KV cache: QK-norm + RoPE + quantising store, then the
                 * int8-cache attention (dpuf_engine.c:1800-1806, 595-752) */
                const DpufKvQ8 c8 = slot_q8(e, e->active, l);
                dpuf_hip_qk_rope_kv(s, M, e->q, e->k, e->v, e->d_norm[4 * l + 1], e->d_norm[4 * l + 2], eps,
                                    e->d_cos, e->d_sin, NULL, NULL, e->d_pos0, e->nq, e->nkv, e->hd, e->max_seq, &c8);
                const DpufWarm wq = attn_warm_fed_o(e, &lj, ln);
                dpuf_hip_attn_q8(s, M, e->capturing ? e->cap_lmax : e->host_pos0 + M, e->q, c8, e->ao, e->scores,
                                 e->d_pos0, e->nq, e->nkv, e->hd, e->max_seq, scale, M == 1 ? &wq : NULL);
                if (M > 1) dpuf_hip_prep(s, M, e->qd, e->ao, W[W_O].sign, e->prep[0]);
                o_prep = M == 1;
                fused = 1;
            } else if (M == 1 && e->host_pos0 + 1 <= ATT_SPLIT_MIN)
                fused = dpuf_hip_attn_dec(s, 1, e->q, e->k, e->v, e->d_norm[4 * l + 1], e->d_norm[4 * l + 2], eps,
                                          e->d_cos, e->d_sin, kc, vc, e->d_pos0, e->nq, e->nkv, e->hd, e->max_seq,
                                          scale, e->ao, W[W_O].sign, e->prep[0], NULL, NULL, 0,
                                          attn_warm(e, &lj, ln)) == 0;
            if (!fused) {
                const int32_t lmax = e->capturing ? e->cap_lmax : e->host_pos0 + M;
                /* the O-input prep rides with the last attention kernel when
                 * it can; otherwise it is a launch of its own */
                int32_t prepped = 0;
                /* one token: QK-norm, RoPE and the KV store inside the scores
                 * launch when the wide kernels apply; their P.V launch warms
                 * the caches for the GEMVs after it */
                const DpufWarm wd = attn_warm_fed_o(e, &lj, ln);
                const int rope_done =
                    M == 1 && dpuf_hip_attn_decode_rope(s, lmax, e->q, e->k, e->v, e->d_norm[4 * l + 1],
                                                        e->d_norm[4 * l + 2], eps, e->d_cos, e->d_sin, kc, vc, e->ao,
                                                        e->scores, e->d_pos0, e->nq, e->nkv, e->hd, e->max_seq,
                                                        scale, &wd) == 0;
                if (!rope_done) {
                    dpuf_hip_qk_rope_kv(s, M, e->q, e->k, e->v, e->d_norm[4 * l + 1], e->d_norm[4 * l + 2], eps,
                                        e->d_cos, e->d_sin, kc, vc, e->d_pos0, e->nq, e->nkv, e->hd, e->max_seq, NULL);
                    if (dpuf_hip_attn_split(s, M, lmax, e->q, kc, vc, e->ao, e->scores, e->d_pos0, e->nq, e->nkv,
                                            e->hd, e->max_seq, scale, W[W_O].sign, e->prep[0], &prepped) != 0)
                        dpuf_hip_attn(s, M, e->q, kc, vc, e->ao, e->scores, e->d_pos0, e->nq, e->nkv, e->hd,
                                      e->max_seq, scale);
                }
                /* one row: the O launch preps its own input (below) */
                if (!prepped && M > 1) dpuf_hip_prep(s, M, e->qd, e->ao, W[W_O].sign, e->prep[0]);
                o_prep = !prepped && M == 1;
            }
            tm_end(e, tm);
        }
        {
            const DpufGemvJob j = jo;
            const int tm5 = tm_begin(e, K_O, gemv_bytes(&W[W_O], 0, n_tiles_of(&W[W_O]), M));
            /* a pending O-input prep runs inside the O launch when it can */
            if (!o_prep || dpuf_hip_swiglu_gemv(s, e->qd, e->ao, NULL, 0.0f, W[W_O].sign, &j,
                                                e->d_pflag + (size_t)l * 1024, e->d_serial) != 0) {
                if (o_prep) dpuf_hip_prep(s, M, e->qd, e->ao, W[W_O].sign, e->prep[0]);
                dpuf_hip_gemv(s, M, 1, &j, NULL, 0.0f);
            }
            tm_end(e, tm5);
        }
        /* (6) h += O; FFN RMSNorm; prep of gate/up input */
        {
            int32_t np = qi[4] ? 2 : 1;
            const uint8_t* ps[2] = {W[W_GATE].sign, W[W_UP].sign};
            const int tm6 = tm_begin(e, K_PREP, 0);
            float* ho = h_other(e);
            dpuf_hip_resnorm_prep(s, M, H, e->hcur, e->hn, ho, e->d_norm[4 * l + 3], eps, np, ps, e->prep, NULL);
            e->hcur = ho;
            tm_end(e, tm6);
        }
        /* (7) gate + up in one launch; with 2 .. 8 or more than 16 rows and
         * one shared input, the launch also runs (8), SwiGLU + prep of the
         * down input, into prep[1] (free: gate and up read prep[0]) */
        int swi = 0;
        {
            const DpufGemvJob* js = jgu;
            double b = gemv_bytes(&W[W_GATE], 0, n_tiles_of(&W[W_GATE]), M) + gemv_bytes(&W[W_UP], 0, n_tiles_of(&W[W_UP]), M);
            const int tm7 = tm_begin(e, K_GU, b);
            if (M > 1 && js[0].p.h == e->prep[0].h && js[1].p.h == e->prep[0].h)
                swi = (M > 8 ? dpuf_hip_gemm_swiglu : dpuf_hip_mvt_swiglu)(s, M, js, e->deadzone, W[W_DOWN].sign,
                                                                         e->prep[1]) == 0;
            if (!swi) dpuf_hip_gemv(s, M, 2, js, NULL, 0.0f);
            tm_end(e, tm7);
        }
        /* (8) SwiGLU + dead zone + prep of the down input, (9) down
         * projection, pruned to keep_tiles with the rest zeroed
         * (dpuf_engine.c:2018-2044).  One row, nothing pruned: one launch
         * whose producer workgroups run (8) while the GEMV workgroups stream
         * their weights. */
        {
            int32_t nt = n_tiles_of(&W[W_DOWN]);
            int32_t kt = (keep_tiles > 0 && keep_tiles < nt) ? keep_tiles : nt;
            DpufGemvJob j = lj.down;
            if (swi) j.p = e->prep[1];
            int fused = 0;
            if (M == 1 && kt == nt) {
                const int tm9 = tm_begin(e, K_DOWN, gemv_bytes(&W[W_DOWN], 0, kt, M));
                fused = dpuf_hip_swiglu_gemv(s, I, e->gate, e->up, e->deadzone, W[W_DOWN].sign, &j,
                                             e->d_pflag + (size_t)l * 1024 + 512, e->d_serial) == 0;
                tm_end(e, tm9);
            }
            if (!fused) {
                if (!swi) {
                    const int tm8 = tm_begin(e, K_PREP, 0);
                    dpuf_hip_swiglu_prep(s, M, I, e->gate, e->up, e->deadzone, W[W_DOWN].sign, e->prep[0]);
                    tm_end(e, tm8);
                }
                const int tm9 = tm_begin(e, K_DOWN, gemv_bytes(&W[W_DOWN], 0, kt, M));
                if (kt < nt)
                    dpuf_hip_gemv_zero(s, M, &j, kt * 16, W[W_DOWN].rows);
                else
                    dpuf_hip_gemv(s, M, 1, &j, NULL, 0.0f);
                tm_end(e, tm9);
            }
        }
        if (e->capture && M <= e->capture_cap)
            dpuf_hip_capture(s, M, H, e->hcur, e->hn, e->capture + (size_t)l * e->capture_cap * H);
    }
}

/* Final residual + output RMSNorm + LM head (with the optional Zone-A early
 * exit) and the device argmax; reads the residual stream h (+ hn).  Returns
 * bit 0: the early-exit flag was computed; bit 1: the step's result words
 * are already published (a one-row argmax step: the LM-head GEMV's chains
 * write partials that one workgroup merges, publishing the token). */
static int enqueue_head(Engine* e, int32_t M, int32_t only_last, int32_t early_tiles, float early_margin,
                        int32_t want_argmax, float* lm_host) {
    void* s = e->stream;
    const int32_t H = e->H;
    const float eps = e->cfg.rms_eps;
    if (only_last == 2) return 0;
    const int32_t lm0 = only_last ? M - 1 : 0, lmM = M - lm0;
    const int32_t nt = n_tiles_of(&e->lm);
    {
        const uint8_t* ps[1] = {e->lm.sign};
        const int tm10 = tm_begin(e, K_PREP, 0);
        dpuf_hip_resnorm_prep(s, lmM, H, e->hcur + (size_t)lm0 * H, e->L > 0 ? e->hn + (size_t)lm0 * H : NULL,
                              h_other(e) + (size_t)lm0 * H, e->d_out_norm, eps, 1, ps, e->prep, NULL);
        tm_end(e, tm10);
    }
    if (head_early(e, lmM, early_tiles)) {
        /* Zone-A early exit (dpuf_engine.c:2091-2136): zone tiles, top-2
         * margin test on the device, then either the -1e9 fill or the
         * remaining tiles, decided by a device flag (no host round trip). */
        int32_t za = early_tiles < 256 ? 256 : early_tiles;
        if (za > nt) za = nt;
        int32_t nz = za * 16 < e->V ? za * 16 : e->V;
        /* the partials of one launch are merged before the next launch
         * writes its own over them */
        void* zone = (char*)e->d_lmred + (size_t)LM_RED_CAP * 16;
        DpufGemvJob j0 = job(&e->lm, 0, za, e->prep[0], e->logits, e->V);
        const int tm11 = tm_begin(e, K_LM, gemv_bytes(&e->lm, 0, za, 1));
        const int32_t n0 = dpuf_hip_gemv_red(s, &j0, NULL, 0.0f, e->d_lmred, LM_RED_CAP);
        dpuf_hip_lm_zone(s, e->d_lmred, n0 > 0 ? n0 : 0, early_margin, e->d_flag, zone);
        int32_t n1 = 0;
        if (za < nt) {
            DpufGemvJob j1 = job(&e->lm, za, nt, e->prep[0], e->logits, e->V);
            n1 = dpuf_hip_gemv_red(s, &j1, e->d_flag, -1e9f, e->d_lmred, LM_RED_CAP);
        }
        tm_end(e, tm11);
        if (want_argmax) {
            dpuf_hip_lm_argmax_publish(s, e->d_lmred, n1 > 0 ? n1 : 0, zone, -1e9f, nz < e->V ? nz : -1, e->logits,
                                       e->d_flag, 1, e->h_io + IO_OUT);
            return 3;
        }
        return 1;
    }
    DpufGemvJob j = job(&e->lm, 0, nt, e->prep[0], lm_host && lmM == 1 ? lm_host : e->logits, e->V);
    const int tm12 = tm_begin(e, K_LM, gemv_bytes(&e->lm, 0, nt, lmM));
    if (want_argmax && lmM == 1 && !lm_host) {
        const int32_t n = dpuf_hip_gemv_red(s, &j, NULL, 0.0f, e->d_lmred, LM_RED_CAP);
        tm_end(e, tm12);
        dpuf_hip_lm_argmax_publish(s, e->d_lmred, n > 0 ? n : 0, NULL, 0.0f, -1, e->logits, e->d_flag, 0,
                                   e->h_io + IO_OUT);
        return 2;
    }
    dpuf_hip_gemv(s, lmM, 1, &j, NULL, 0.0f);
    tm_end(e, tm12);
    if (want_argmax) dpuf_hip_argmax(s, e->logits + (size_t)(lmM - 1) * e->V, e->V, e->d_tok, e->d_red);
    return 0;
}

static int32_t forward_common(Engine* e, int32_t n_tokens, const int32_t* token_ids, int32_t pos0,
                              const float* embeds_in, const int32_t* pos_t, const int32_t* pos_h,
                              const int32_t* pos_w, const float* const* deepstack_in, int32_t only_last,
                              float* logits_out, int32_t* token_out, int32_t use_graph) {
    if (!e || (!token_ids && !embeds_in) || (!logits_out && !token_out && only_last != 2)) return -1;
    if (n_tokens <= 0 || n_tokens > DPUF_AMD_MAX_BATCH) return -2;
    if (pos0 < 0 || pos0 + n_tokens > e->max_seq) return -3;
    if (deepstack_in) return -5;
    if (pos_t || pos_h || pos_w) {
        for (int32_t m = 0; m < n_tokens; m++) {
            int32_t p = pos0 + m;
            if ((pos_t && pos_t[m] != p) || (pos_h && pos_h[m] != p) || (pos_w && pos_w[m] != p)) return -5;
        }
    }
    for (int32_t m = 0; m < n_tokens; m++) {
        int32_t id = token_ids ? token_ids[m] : -1;
        if (id >= e->V || (id < 0 && !embeds_in)) return -4;
    }
    const int32_t M = n_tokens;
    begin_call(e);
    int32_t keep = 0, early = 0;
    env_int(M > 1 ? "DPUF_PREFILL_KEEP_TILES" : "DPUF_GEN_KEEP_TILES", &keep);
    int32_t has_early = env_int("DPUF_EARLY_TILES", &early);
    const char* em = getenv("DPUF_EARLY_MARGIN");
    float margin = em ? (float)atof(em) : 1.25f;
    if (!has_early) early = 0;
    else if (early <= 0) early = 1; /* env set: the zone is at least 256 tiles */

    /* the embedding kernel reads ids and pos0 from h_io (no copy) */
    volatile int32_t* io = e->h_io;
    for (int32_t m = 0; m < M; m++) io[m] = token_ids ? token_ids[m] : -1;
    io[IO_POS] = pos0;
    io[IO_POS + 1] = next_serial(e);
    /* one row: the embedding kernel reads the hidden state from h_emb (no
     * copy, graphs replay it); more rows go to the device first */
    if (embeds_in && M == 1) memcpy(e->h_emb, embeds_in, (size_t)e->H * 4);
    else if (embeds_in) dpuf_hip_h2d(e->embeds, embeds_in, (size_t)M * e->H * 4, e->stream);
    /* a one-row LM head whose logits go to the host writes them to h_logits
     * itself (the same for every step of a graph key: want_argmax clear and
     * only_last != 2 imply logits_out) */
    const int32_t want_argmax = token_out != NULL;
    const int32_t lm_rows = only_last ? 1 : M;
    float* lm_host = only_last != 2 && logits_out && !want_argmax && lm_rows == 1 && !head_early(e, 1, early)
                         ? e->h_logits
                         : NULL;

    const int tm13 = tm_begin(e, K_CALL, (double)e->weight_bytes);
    const int graphable = use_graph && !e->no_graphs && M == 1 && !e->timing && !e->capture;
    e->host_pos0 = pos0;
    e->capturing = 0;
    if (graphable) {
        const int32_t bucket = attn_bucket(e, pos0 + 1);
        int32_t key[7] = {only_last, keep, early, e->active, 0, bucket, want_argmax};
        memcpy(&key[4], &margin, 4);
        int gi = -1;
        for (int i = 0; i < N_GRAPHS && gi < 0; i++)
            if (e->graphs[i] && memcmp(key, e->graph_keys[i], sizeof key) == 0) gi = i;
        if (gi < 0) {
            /* a free entry, else the least recently used */
            gi = 0;
            for (int i = 0; i < N_GRAPHS; i++) {
                if (!e->graphs[i]) { gi = i; break; }
                if (e->graph_used[i] < e->graph_used[gi]) gi = i;
            }
            dpuf_hip_graph_destroy(e->graphs[gi]);
            e->graphs[gi] = NULL;
            if (dpuf_hip_capture_begin(e->stream) == 0) {
                e->capturing = 1;
                e->cap_lmax = bucket;
                enqueue_forward(e, 1, 0, only_last, keep, early, margin, want_argmax, lm_host);
                e->capturing = 0;
                e->graphs[gi] = dpuf_hip_capture_end(e->stream);
                memcpy(e->graph_keys[gi], key, sizeof key);
            }
        }
        if (e->graphs[gi]) {
            e->graph_used[gi] = ++e->graph_tick;
            dpuf_hip_graph_launch(e->graphs[gi], e->stream);
        } else {
            enqueue_forward(e, M, 0, only_last, keep, early, margin, want_argmax, lm_host);
        }
    } else {
        enqueue_forward(e, M, embeds_in != NULL, only_last, keep, early, margin, want_argmax, lm_host);
    }
    tm_end(e, tm13);
    if (only_last != 2 && logits_out && !lm_host)
        dpuf_hip_d2h(logits_out, e->logits, (size_t)lm_rows * e->V * 4, e->stream);
    if (dpuf_hip_sync(e->stream) != 0) return -6;
    tm_collect(e);
    const int32_t flag = io[IO_OUT], tok = io[IO_OUT + 1];
    const int32_t rc = end_call(e, io[IO_OUT + 2]);
    if (rc == 0 && only_last != 2) {
        if (lm_host) memcpy(logits_out, e->h_logits, (size_t)e->V * 4);
        if (flag) e->early_exits++;
        if (token_out) *token_out = tok;
    }
    return rc;
}

DPUF_EXPORT int32_t dpuf_engine_forward_batch_ex(void* handle, int32_t n_tokens, const int32_t* token_ids,
                                                 int32_t pos0, const float* embeds_in, const int32_t* pos_t,
                                                 const int32_t* pos_h, const int32_t* pos_w,
                                                 const float* const* deepstack_in, int32_t only_last_logits,
                                                 float* logits_out) {
    Engine* e = (Engine*)handle;
    if (!e || (!logits_out && only_last_logits != 2)) return -1;
    /* one-token steps replay a captured graph (forward_common decides) */
    return forward_common(e, n_tokens, token_ids, pos0, embeds_in, pos_t, pos_h, pos_w, deepstack_in,
                          only_last_logits, logits_out, NULL, 1);
}

DPUF_EXPORT int32_t dpuf_engine_forward_batch(void* handle, int32_t n_tokens, const int32_t* token_ids, int32_t pos0,
                                              int32_t only_last_logits, float* logits_out) {
    return dpuf_engine_forward_batch_ex(handle, n_tokens, token_ids, pos0, NULL, NULL, NULL, NULL, NULL,
                                        only_last_logits, logits_out);
}

DPUF_EXPORT int32_t dpuf_engine_forward_token(void* handle, int32_t token_id, int32_t pos, float* logits_out) {
    int32_t t = token_id;
    return dpuf_engine_forward_batch(handle, 1, &t, pos, 1, logits_out);
}

/* One next token for each of n sessions in one pass: token_ids[i] goes into
 * session slot_ids[i] (distinct) at positions[i], every row of every GEMM
 * serves all n.  Per token the arithmetic is the one-token decode's, with the
 * decode keep-tiles setting and no Zone-A early exit. */
DPUF_EXPORT int32_t dpuf_amd_engine_forward_slots(void* handle, int32_t n, const int32_t* slot_ids,
                                                  const int32_t* token_ids, const int32_t* positions,
                                                  float* logits_out, int32_t* tokens_out) {
    Engine* e = (Engine*)handle;
    if (!e || n <= 0 || !slot_ids || !token_ids || !positions || (!logits_out && !tokens_out)) return -1;
    if (n > DPUF_AMD_MAX_BATCH) return -2;
    if (e->hd != 64 && e->hd != 128 && e->hd != 256) return -5;
    for (int32_t i = 0; i < n; i++) {
        if (slot_ids[i] < 0 || slot_ids[i] >= N_SLOTS) return -1;
        for (int32_t j = 0; j < i; j++)
            if (slot_ids[j] == slot_ids[i]) return -1;
        if (positions[i] < 0 || positions[i] + 1 > e->max_seq) return -3;
        if (token_ids[i] < 0 || token_ids[i] >= e->V) return -4;
        if (!slot_alloc(e, slot_ids[i])) return -2;
    }
    /* batch order: sessions the fused decode attention serves (fp32 cache,
     * at most DPUF_HIP_DEC_MAX_KEYS keys) first, the others after them;
     * ord[m] is the caller's index of batch row m */
    int32_t* ord = (int32_t*)malloc((size_t)n * sizeof(int32_t));
    float* lg = logits_out ? (float*)malloc((size_t)n * e->V * sizeof(float)) : NULL;
    if (!ord || (logits_out && !lg)) {
        free(ord);
        free(lg);
        return -2;
    }
    int32_t ns = 0;
    for (int32_t pass = 0; pass < 2; pass++)
        for (int32_t i = 0; i < n; i++) {
            const int shrt = !is_q8(e) && positions[i] + 1 <= ATT_SPLIT_MIN;
            if (shrt == (pass == 0)) ord[ns++] = i;
        }
    ns = 0;
    while (ns < n && !is_q8(e) && positions[ord[ns]] + 1 <= ATT_SPLIT_MIN) ns++;
    begin_call(e);
    volatile int32_t* io = e->h_io;
    float** hk = (float**)e->h_ms;
    int32_t* hpos = (int32_t*)(hk + 2 * DPUF_AMD_MAX_BATCH);
    for (int32_t m = 0; m < n; m++) {
        const int32_t i = ord[m];
        hk[m] = is_q8(e) ? NULL : slot_k(e, slot_ids[i]);
        hk[DPUF_AMD_MAX_BATCH + m] = is_q8(e) ? NULL : slot_v(e, slot_ids[i]);
        hpos[m] = positions[i];
        e->ms_slot[m] = slot_ids[i];
        e->ms_pos[m] = positions[i];
        io[m] = token_ids[i];
    }
    io[IO_POS] = 0;
    io[IO_POS + 1] = next_serial(e);
    /* the tables in one copy (the device layout: d_ms_vc and d_ms_pos follow
     * d_ms_kc) */
    dpuf_hip_h2d(e->d_ms_kc, e->h_ms, (size_t)2 * DPUF_AMD_MAX_BATCH * sizeof(float*) + (size_t)n * 4, e->stream);
    int32_t keep = 0;
    env_int("DPUF_GEN_KEEP_TILES", &keep);
    e->ms_n = n;
    e->ms_short = ns;
    e->capturing = 0;
    const int tm = tm_begin(e, K_CALL, (double)e->weight_bytes);
    enqueue_forward(e, n, 0, 0, keep, 0, 1.25f, 0, NULL);
    e->ms_n = 0;
    e->ms_short = 0;
    if (tokens_out) dpuf_hip_argmax_rows(e->stream, e->logits, e->V, n, e->d_ms_tok, e->h_tok, e->d_lmred);
    tm_end(e, tm);
    if (logits_out) dpuf_hip_d2h(lg, e->logits, (size_t)n * e->V * 4, e->stream);
    const int32_t rc = dpuf_hip_sync(e->stream);
    tm_collect(e);
    int32_t out = rc != 0 ? -6 : end_call(e, io[IO_OUT + 2]);
    if (out == 0) {
        for (int32_t m = 0; m < n; m++) {
            if (logits_out) memcpy(logits_out + (size_t)ord[m] * e->V, lg + (size_t)m * e->V, (size_t)e->V * 4);
            if (tokens_out) tokens_out[ord[m]] = ((volatile int32_t*)e->h_tok)[m];
        }
    }
    free(ord);
    free(lg);
    return out;
}

DPUF_EXPORT int32_t dpuf_amd_engine_forward_argmax(void* handle, int32_t n_tokens, const int32_t* token_ids,
                                                   int32_t pos0, const float* embeds_in, int32_t use_graph,
                                                   int32_t* token_out, float* logits_out) {
    Engine* e = (Engine*)handle;
    if (!e || !token_out) return -1;
    return forward_common(e, n_tokens, token_ids, pos0, embeds_in, NULL, NULL, NULL, NULL, 1, logits_out, token_out,
                          use_graph);
}

/* ------------------------------------------------------------------------- */
/* Test and measurement hooks (include/dpuf_amd.h)                            */
/* ------------------------------------------------------------------------- */

DPUF_EXPORT int32_t dpuf_amd_engine_set_kv(void* handle, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                                           const float* k, const float* v) {
    Engine* e = (Engine*)handle;
    if (!e || layer < 0 || layer >= e->L || kvh < 0 || kvh >= e->nkv || pos0 < 0 || n < 0 || pos0 + n > e->max_seq ||
        !k || !v)
        return -1;
    dpuf_hip_clear_error();
    size_t off = (((size_t)layer * e->nkv + kvh) * (size_t)e->max_seq + pos0) * e->hd;
    if (is_q8(e)) {
        /* quantised on the device exactly as the KV store does */
        if (n == 0) return 0;
        float* tmp = (float*)dpuf_hip_malloc((size_t)n * e->hd * 8);
        if (!tmp) return -1;
        dpuf_hip_h2d(tmp, k, (size_t)n * e->hd * 4, e->stream);
        dpuf_hip_h2d(tmp + (size_t)n * e->hd, v, (size_t)n * e->hd * 4, e->stream);
        dpuf_hip_q8_rows(e->stream, tmp, tmp + (size_t)n * e->hd, n, e->hd, slot_q8(e, e->active, 0),
                         off / (size_t)e->hd);
        const int32_t rc = dpuf_hip_sync(e->stream);
        dpuf_hip_free(tmp);
        return rc;
    }
    dpuf_hip_h2d(slot_k(e, e->active) + off, k, (size_t)n * e->hd * 4, e->stream);
    dpuf_hip_h2d(slot_v(e, e->active) + off, v, (size_t)n * e->hd * 4, e->stream);
    return dpuf_hip_sync(e->stream);
}

DPUF_EXPORT int32_t dpuf_amd_engine_get_kv(void* handle, int32_t layer, int32_t kvh, int32_t pos0, int32_t n,
                                           float* k, float* v) {
    Engine* e = (Engine*)handle;
    if (!e || layer < 0 || layer >= e->L || kvh < 0 || kvh >= e->nkv || pos0 < 0 || n < 0 || pos0 + n > e->max_seq ||
        !k || !v)
        return -1;
    dpuf_hip_clear_error();
    size_t off = (((size_t)layer * e->nkv + kvh) * (size_t)e->max_seq + pos0) * e->hd;
    if (is_q8(e)) { /* dequantised: q * scale */
        if (n == 0) return 0;
        float* tmp = (float*)dpuf_hip_malloc((size_t)n * e->hd * 8);
        if (!tmp) return -1;
        dpuf_hip_q8_dequant(e->stream, slot_q8(e, e->active, 0), off, (size_t)n * e->hd, tmp,
                            tmp + (size_t)n * e->hd);
        dpuf_hip_d2h(k, tmp, (size_t)n * e->hd * 4, e->stream);
        dpuf_hip_d2h(v, tmp + (size_t)n * e->hd, (size_t)n * e->hd * 4, e->stream);
        const int32_t rc = dpuf_hip_sync(e->stream);
        dpuf_hip_free(tmp);
        return rc;
    }
    dpuf_hip_d2h(k, slot_k(e, e->active) + off, (size_t)n * e->hd * 4, e->stream);
    dpuf_hip_d2h(v, slot_v(e, e->active) + off, (size_t)n * e->hd * 4, e->stream);
    return dpuf_hip_sync(e->stream);
}

DPUF_EXPORT int32_t dpuf_amd_engine_set_capture(void* handle, int32_t max_tokens) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || max_tokens < 0 || max_tokens > DPUF_AMD_MAX_BATCH) return -1;
    dpuf_hip_free(e->capture);
    e->capture = NULL;
    e->capture_cap = 0;
    if (max_tokens == 0 || e->L == 0) return 0;
    e->capture = (float*)dpuf_hip_malloc((size_t)e->L * max_tokens * e->H * 4);
    if (!e->capture) return -1;
    e->capture_cap = max_tokens;
    dpuf_hip_fill_zero(e->capture, (size_t)e->L * max_tokens * e->H * 4, e->stream);
    return dpuf_hip_sync(e->stream);
}

DPUF_EXPORT int32_t dpuf_amd_engine_get_capture(void* handle, float* out, size_t n_floats) {
    dpuf_hip_clear_error();
    Engine* e = (Engine*)handle;
    if (!e || !e->capture || !out) return -1;
    size_t total = (size_t)e->L * e->capture_cap * e->H;
    if (n_floats > total) n_floats = total;
    dpuf_hip_d2h(out, e->capture, n_floats * 4, e->stream);
    return dpuf_hip_sync(e->stream);
}

DPUF_EXPORT void dpuf_amd_engine_set_graphs(void* handle, int32_t enable) {
    Engine* e = (Engine*)handle;
    if (!e) return;
    e->no_graphs = enable ? 0 : 1;
    if (e->no_graphs) {
        for (int i = 0; i < N_GRAPHS; i++) {
            dpuf_hip_graph_destroy(e->graphs[i]);
            e->graphs[i] = NULL;
        }
    }
}

DPUF_EXPORT void dpuf_amd_engine_set_timing(void* handle, int32_t enable) {
    Engine* e = (Engine*)handle;
    if (!e) return;
    e->timing = enable ? 1 : 0;
    e->n_ev = 0;
    memset(e->t_ms, 0, sizeof e->t_ms);
    memset(e->t_cnt, 0, sizeof e->t_cnt);
    memset(e->t_bytes, 0, sizeof e->t_bytes);
}

DPUF_EXPORT int32_t dpuf_amd_engine_get_timing(void* handle, int32_t kind, double* total_ms, int64_t* count,
                                               double* bytes) {
    Engine* e = (Engine*)handle;
    if (!e || kind < 0 || kind >= N_KINDS) return -1;
    if (total_ms) *total_ms = e->t_ms[kind];
    if (count) *count = e->t_cnt[kind];
    if (bytes) *bytes = e->t_bytes[kind];
    return 0;
}

DPUF_EXPORT uint64_t dpuf_amd_engine_weight_bytes(void* handle) {
    Engine* e = (Engine*)handle;
    return e ? e->weight_bytes : 0;
}

DPUF_EXPORT int64_t dpuf_amd_engine_early_exit_count(void* handle) {
    Engine* e = (Engine*)handle;
    return e ? e->early_exits : 0;
}

DPUF_EXPORT int64_t dpuf_amd_attn_path_count(int32_t which) { return dpuf_hip_attn_path_count(which); }

/* Jobs of one GEMV launch of kind `which` in layer l (see dpuf_amd_gemv_bench). */
static int32_t bench_jobs(Engine* e, int32_t which, int32_t l, DpufGemvJob* js, double* bytes, int32_t M) {
    static const int32_t mats[2][3] = {{W_GATE, W_UP, -1}, {W_Q, W_K, W_V}};
    if (which == 7) {
        js[0] = job(&e->lm, 0, n_tiles_of(&e->lm), e->prep[0], e->logits, e->lm.rows);
        *bytes = gemv_bytes(&e->lm, 0, n_tiles_of(&e->lm), M);
        return 1;
    }
    const DpufDevW* W = e->lw + (size_t)l * 7;
    if (which < 7) {
        js[0] = job(&W[which], 0, n_tiles_of(&W[which]), e->prep[0], e->up, W[which].rows);
        *bytes = gemv_bytes(&W[which], 0, n_tiles_of(&W[which]), M);
        return 1;
    }
    const int32_t* ms = mats[which - 8];
    float* outs[3] = {e->gate, e->up, e->v};
    if (which == 9) {
        outs[0] = e->q;
        outs[1] = e->k;
    }
    int32_t n = 0;
    *bytes = 0.0;
    for (int k = 0; k < 3 && ms[k] >= 0; k++, n++) {
        const DpufDevW* w = &W[ms[k]];
        js[k] = job(w, 0, n_tiles_of(w), e->prep[0], outs[k], w->rows);
        *bytes += gemv_bytes(w, 0, n_tiles_of(w), M);
    }
    return n;
}

DPUF_EXPORT double dpuf_amd_gemv_bench(void* handle, int32_t which, int32_t M, int32_t iters, int32_t start_layer,
                                       double* bytes) {
    Engine* e = (Engine*)handle;
    if (!e || which < 0 || which > 9 || M < 1 || iters < 1) return -1.0;
    if (which != 7 && (e->L == 0 || start_layer < 0 || start_layer >= e->L)) return -1.0;
    if (M > DPUF_AMD_MAX_BATCH) return -1.0;
    begin_call(e);
    DpufGemvJob js[3];
    double b0 = 0.0;
    bench_jobs(e, which, start_layer, js, &b0, M);
    const int32_t K = js[0].w.cols;
    /* activations: the prep of a fixed, non-trivial vector per row */
    float* x = (float*)malloc((size_t)M * K * 4);
    if (!x) return -1.0;
    uint32_t st = 12345u;
    for (size_t i = 0; i < (size_t)M * K; i++) {
        st = st * 1664525u + 1013904223u;
        x[i] = ((float)(st >> 8) / 16777216.0f) * 2.0f - 1.0f;
    }
    float* dx = (float*)dpuf_hip_malloc((size_t)M * K * 4);
    if (!dx) {
        free(x);
        return -1.0;
    }
    dpuf_hip_h2d(dx, x, (size_t)M * K * 4, e->stream);
    dpuf_hip_prep(e->stream, M, K, dx, js[0].w.sign, e->prep[0]);
    dpuf_hip_sync(e->stream);
    dpuf_hip_free(dx);
    free(x);
    void* a = dpuf_hip_event_create();
    void* b = dpuf_hip_event_create();
    const int32_t nl = which == 7 ? 1 : e->L - start_layer;
    int32_t n = bench_jobs(e, which, start_layer, js, &b0, M);
    dpuf_hip_gemv(e->stream, M, n, js, NULL, 0.0f); /* warm-up launch */
    dpuf_hip_event_record(a, e->stream);
    for (int32_t i = 0; i < iters; i++) {
        double bb;
        n = bench_jobs(e, which, start_layer + (i % nl), js, &bb, M);
        dpuf_hip_gemv(e->stream, M, n, js, NULL, 0.0f);
    }
    dpuf_hip_event_record(b, e->stream);
    float ms = dpuf_hip_event_elapsed_ms(a, b);
    dpuf_hip_event_destroy(a);
    dpuf_hip_event_destroy(b);
    if (bytes) *bytes = b0;
    int32_t* hp = e->h_pinned;
    dpuf_hip_d2h(hp + 3, e->d_err, 4, e->stream);
    if (dpuf_hip_sync(e->stream) != 0 || end_call(e, hp[3]) != 0) return -1.0;
    return (double)ms / iters;
}

DPUF_EXPORT void dpuf_amd_set_gemv_max_workgroups(int32_t n) { dpuf_hip_set_gemv_max_wg(n); }

DPUF_EXPORT int32_t dpuf_amd_reduce_check(const float* x, int32_t n, int32_t offset, int32_t mode, float thr) {
    dpuf_hip_clear_error();
    if (!x || n < 1 || offset < 0 || offset > 3 || (mode != 0 && mode != 1) || dpuf_hip_device_count() <= 0)
        return -1;
    void* s = dpuf_hip_stream_create();
    float* d = (float*)dpuf_hip_malloc(((size_t)n + 4) * 4);
    void* red = dpuf_hip_malloc(DPUF_HIP_RED_SCRATCH);
    int32_t* o = (int32_t*)dpuf_hip_malloc(4);
    int32_t r = -1;
    if (s && d && red && o) {
        dpuf_hip_h2d(d + offset, x, (size_t)n * 4, s);
        if (mode == 1) dpuf_hip_argmax(s, d + offset, n, o, red);
        else dpuf_hip_topcheck(s, d + offset, n, thr, o, red);
        dpuf_hip_d2h(&r, o, 4, s);
        if (dpuf_hip_sync(s) != 0 || !dpuf_hip_ok()) r = -1;
    }
    dpuf_hip_free(o);
    dpuf_hip_free(red);
    dpuf_hip_free(d);
    if (s) dpuf_hip_stream_destroy(s);
    return r;
}

DPUF_EXPORT int32_t dpuf_amd_reduce_check_noalloc(const float* d_x, int32_t n, int32_t mode, float thr,
                                                  int32_t* d_out, void* hip_stream) {
    dpuf_hip_clear_error();
    if (!d_x || !d_out || (mode != 0 && mode != 1)) return -1;
    if (n < 1 || n > DPUF_AMD_NOALLOC_MAX_N) return -2;
    return dpuf_hip_reduce_noalloc(d_x, n, mode, thr, d_out, hip_stream);
}

DPUF_EXPORT double dpuf_amd_copy_bench(size_t bytes, int32_t iters) {
    dpuf_hip_clear_error();
    if (bytes == 0 || iters < 1 || dpuf_hip_device_count() <= 0) return -1.0;
    void* s = dpuf_hip_stream_create();
    void* src = dpuf_hip_malloc(bytes);
    void* dst = dpuf_hip_malloc(bytes);
    double r = -1.0;
    if (s && src && dst) {
        dpuf_hip_fill_zero(src, bytes, s);
        dpuf_hip_d2d(dst, src, bytes, s);
        void* a = dpuf_hip_event_create();
        void* b = dpuf_hip_event_create();
        dpuf_hip_event_record(a, s);
        for (int32_t i = 0; i < iters; i++) dpuf_hip_d2d(dst, src, bytes, s);
        dpuf_hip_event_record(b, s);
        r = dpuf_hip_event_elapsed_ms(a, b) / iters;
        dpuf_hip_event_destroy(a);
        dpuf_hip_event_destroy(b);
        if (!dpuf_hip_ok()) r = -1.0;
    }
    dpuf_hip_free(src);
    dpuf_hip_free(dst);
    if (s) dpuf_hip_stream_destroy(s);
    return r;
}
