/*
 * drive.c -- the host C of this repository (the .dpuf packer, container
 * writer and reader with its JSON header parser and tile verify / heal, the
 * CRC helpers, and the oracle) exercised under AddressSanitizer and
 * UndefinedBehaviorSanitizer.  Built and run by tests/test_cpu_sanitize.py:
 *
 *   drive <dir>
 *
 * Builds a mode 12 model and a had4p-hybrid (modes 13 / 14) model, writes
 * both as containers, reopens them with verification, runs the oracle on
 * them (fp32 and int8 KV caches), then reopens ~400 damaged copies of the
 * mode 12 container: truncations, flipped tile bytes, and JSON headers
 * mutated byte by byte with the header CRC recomputed so the parser itself
 * sees the malformed text.  Any sanitizer report aborts the run; exit 0
 * means every path ran clean.  Mutations and tokens come from a fixed seed.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../dpuf_amd/csrc/dpuf_tools.h"
#include "../../oracle/oracle.h"

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
    rs ^= rs << 13;
    rs ^= rs >> 7;
    rs ^= rs << 17;
    return (uint32_t)(rs >> 11);
}

static uint8_t* slurp(const char* path, size_t* n) {
    FILE* f = fopen(path, "rb");
    if (!f) return NULL;
    fseek(f, 0, SEEK_END);
    long len = ftell(f);
    fseek(f, 0, SEEK_SET);
    uint8_t* b = (uint8_t*)malloc((size_t)len);
    if (b && fread(b, 1, (size_t)len, f) != (size_t)len) {
        free(b);
        b = NULL;
    }
    fclose(f);
    *n = (size_t)len;
    return b;
}

static int spit(const char* path, const uint8_t* b, size_t n) {
    FILE* f = fopen(path, "wb");
    if (!f) return 0;
    int ok = fwrite(b, 1, n, f) == n;
    fclose(f);
    return ok;
}

/* Prefill + greedy decode on the oracle; returns the last greedy id. */
static int run_oracle(const DpufToolsModel* m, int kv_type) {
    DpufModelConfig cfg = *dpuf_tools_model_cfg(m);
    cfg.kv_type = kv_type;
    OrcEngine* e = orc_engine_create(&cfg, dpuf_tools_model_layers(m), dpuf_tools_model_tok(m),
                                     dpuf_tools_model_lm(m), dpuf_tools_model_out_norm(m));
    if (!e) return -1;
    const int V = cfg.vocab_size;
    float* lg = (float*)malloc((size_t)V * 8 * sizeof(float));  /* all 8 prefill rows */
    int32_t ids[8];
    for (int i = 0; i < 8; i++) ids[i] = (int32_t)(rnd() % (uint32_t)V);
    int tok = -1;
    if (orc_engine_forward(e, 8, ids, 0, NULL, 0, lg) == 0) {
        tok = orc_argmax(lg + (size_t)7 * V, V);
        for (int s = 0; s < 3 && tok >= 0; s++) {
            int32_t t = tok;
            if (orc_engine_forward(e, 1, &t, 8 + s, NULL, 1, lg) != 0) tok = -1;
            else tok = orc_argmax(lg, V);
        }
    }
    free(lg);
    orc_engine_destroy(e);
    return tok;
}

int main(int argc, char** argv) {
    if (argc < 2) return 2;
    char p12[1024], phy[1024], pm[1024];
    snprintf(p12, sizeof p12, "%s/m12.dpuf", argv[1]);
    snprintf(phy, sizeof phy, "%s/hybrid.dpuf", argv[1]);
    snprintf(pm, sizeof pm, "%s/mut.dpuf", argv[1]);

    DpufToolsSpec sp;
    memset(&sp, 0, sizeof sp);
    sp.hidden_size = 128;
    sp.intermediate_size = 256;
    sp.num_layers = 2;
    sp.num_q_heads = 4;
    sp.num_kv_heads = 2;
    sp.head_dim = 64;
    sp.vocab_size = 512;
    sp.max_seq_len = 32;
    sp.tie_word_embeddings = 1;
    sp.weight_std = 0.02f;
    sp.rms_eps = 1e-6f;
    sp.rope_theta = 1e6f;
    sp.seed = 77;
    for (int plan = 0; plan < 2; plan++) {
        sp.weight_plan = plan;
        DpufToolsModel* m = dpuf_tools_build_model(&sp);
        if (!m) { fprintf(stderr, "build (plan %d) failed\n", plan); return 1; }
        const char* path = plan ? phy : p12;
        if (dpuf_tools_save_container(m, path) == 0) { fprintf(stderr, "save failed\n"); return 1; }
        rs = 0x9E3779B97F4A7C15ull + (uint64_t)plan;
        const int t0 = run_oracle(m, 0), t1 = run_oracle(m, 1);
        dpuf_tools_free_model(m);
        int st = 0;
        DpufToolsModel* r = dpuf_tools_open_container(path, 1, 0, &st);
        if (!r) { fprintf(stderr, "reopen (plan %d) failed: %d\n", plan, st); return 1; }
        rs = 0x9E3779B97F4A7C15ull + (uint64_t)plan;  /* the same prompts for the reopened model */
        const int u0 = run_oracle(r, 0), u1 = run_oracle(r, 1);
        dpuf_tools_free_model(r);
        printf("plan %d: greedy ids %d %d (built) %d %d (reopened)\n", plan, t0, t1, u0, u1);
        if (t0 < 0 || t1 < 0 || t0 != u0 || t1 != u1) return 1;
    }

    size_t n = 0;
    uint8_t* orig = slurp(p12, &n);
    if (!orig || n < 64) return 1;
    uint32_t hlen, hcrc;
    memcpy(&hcrc, orig + 12, 4);
    memcpy(&hlen, orig + 20, 4);
    const int crc_ok = 24u + (uint64_t)hlen <= n && dpuf_crc32_bytes(orig + 24, hlen) == hcrc;
    printf("container %zu bytes, header %u bytes, header CRC recomputable: %d\n", n, hlen, crc_ok);
    if (!crc_ok) return 1;
    uint8_t* b = (uint8_t*)malloc(n);
    int opened = 0, refused = 0;
    for (int it = 0; it < 400; it++) {
        memcpy(b, orig, n);
        size_t len = n;
        const int kind = it % 4;
        if (kind == 0) {
            len = 24 + rnd() % (uint32_t)(n - 24);  /* truncation */
        } else if (kind == 1) {
            for (int k = 0; k < 1 + (int)(rnd() % 8); k++) b[24 + hlen + rnd() % (uint32_t)(n - 24 - hlen)] ^= (uint8_t)(1 + rnd() % 255);
        } else {
            /* the JSON header: flipped, overwritten or digit bytes, CRC fixed */
            for (int k = 0; k < 1 + (int)(rnd() % 4); k++) {
                const uint32_t o = 24 + rnd() % hlen;
                const uint32_t c = rnd() % 4;
                b[o] = c == 0 ? (uint8_t)(b[o] ^ (1u << (rnd() % 8)))
                     : c == 1 ? (uint8_t)"{}[]\":,-0123456789e"[rnd() % 20]
                     : c == 2 ? (uint8_t)('0' + rnd() % 10)
                              : (uint8_t)0;
            }
            const uint32_t c2 = dpuf_crc32_bytes(b + 24, hlen);
            memcpy(b + 12, &c2, 4);
        }
        if (!spit(pm, b, len)) return 1;
        int st = 0;
        DpufToolsModel* r = dpuf_tools_open_container(pm, 1, 0, &st);
        if (r) {
            opened++;
            const DpufModelConfig* c = dpuf_tools_model_cfg(r);
            /* a header that still parses to the same small shape runs the oracle too */
            if (c->hidden_size == 128 && c->num_layers == 2 && c->vocab_size == 512 && c->max_seq_len == 32 &&
                c->head_dim == 64 && c->num_q_heads == 4 && c->num_kv_heads == 2 && c->intermediate_size == 256)
                (void)run_oracle(r, it & 1);
            dpuf_tools_free_model(r);
        } else {
            refused++;
        }
    }
    printf("damaged containers: %d opened (healed or harmless), %d refused\n", opened, refused);
    free(b);
    free(orig);
    return 0;
}
