/* A CPU stand-in for a backend plugin, used by the driver tests only: it exports the v1
 * and v2 plugin symbols with a hash-based recurrent "model" whose logits the tests can
 * recompute in numpy.  State per stream: a u64 s, zero after a reset; a token t moves
 * it to mix(s * 0x100000001b3 + t + 1); the logits of state s are
 *   l[v] = float((mix(s ^ v * 0x9e3779b97f4a7c15) >> 40) % 4001) / 400 - 5    (f32 ops).
 * The weights file holds the vocabulary size as one little-endian u32.
 * FAKE_PLUGIN_ABI=1 in the environment makes abi_version() report a v1-only plugin.
 * FAKE_PLUGIN_FAIL_AFTER=k makes every forward / forward_batch after the first k
 * (counted since init) fail with FORWARD_FAILED.
 * Built with -DFAKE_PLUGIN_CDF (and linked against libredukt_host.so) it also exports the
 * device-CDF entry points of the GPU library (include/redukt_backend.h), each computing its
 * CDF rows with the host's redukt_cdf_from_logits: forward_batch_cdf, _sym, _find and the
 * queued _sym_submit / _sym_wait (two calls in flight, run at submit). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
    uint32_t ffi_version, vocab_size, hidden_dim;
    uint8_t name[64];
} BackendInfo;

static uint32_t g_vocab;
static uint64_t g_v1;
static uint64_t* g_slot;
static uint32_t g_cap;
static uint64_t g_calls;

/* 1 when this forward call must fail (FAKE_PLUGIN_FAIL_AFTER). */
static int fail_now(void) {
    const char* e = getenv("FAKE_PLUGIN_FAIL_AFTER");
    return e && ++g_calls > (uint64_t)strtoull(e, NULL, 10);
}

static uint64_t mix(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}
static uint64_t step(uint64_t s, uint32_t t) { return mix(s * 0x100000001b3ULL + t + 1); }
static void logits_of(uint64_t s, float* out) {
    for (uint32_t v = 0; v < g_vocab; ++v) {
        const uint64_t h = mix(s ^ ((uint64_t)v * 0x9e3779b97f4a7c15ULL));
        out[v] = (float)((h >> 40) % 4001) / 400.0f - 5.0f;
    }
}

int redukt_backend_init(const uint8_t* path, int32_t dev, BackendInfo* info) {
    (void)dev;
    FILE* f = fopen((const char*)path, "rb");
    if (!f) return 4;
    uint32_t v = 0;
    size_t got = fread(&v, 4, 1, f);
    fclose(f);
    if (got != 1 || v == 0) return 4;
    g_vocab = v;
    g_v1 = 0;
    g_calls = 0;
    if (info) {
        memset(info, 0, sizeof *info);
        info->ffi_version = 1;
        info->vocab_size = v;
        info->hidden_dim = 8;
        strcpy((char*)info->name, "fake-plugin");
    }
    return 0;
}

int redukt_backend_forward(uint32_t tok, float* out, uint32_t vocab) {
    if (vocab != g_vocab || tok >= g_vocab || !out || fail_now()) return 2;
    g_v1 = step(g_v1, tok);
    logits_of(g_v1, out);
    return 0;
}

void redukt_backend_reset_state(void) { g_v1 = 0; }

static void free_queued(void);

void redukt_backend_free(void) {
    free(g_slot);
    g_slot = NULL;
    g_cap = 0;
    free_queued();
}

uint32_t redukt_backend_abi_version(void) {
    const char* e = getenv("FAKE_PLUGIN_ABI");
    return e ? (uint32_t)atoi(e) : 2u;
}

int32_t redukt_backend_batch_init(uint32_t n) {
    if (n == 0) return 5;
    free(g_slot);
    g_slot = (uint64_t*)calloc(n, sizeof(uint64_t));
    g_cap = n;
    return 0;
}

int32_t redukt_backend_batch_reset(const uint32_t* slots, uint32_t n) {
    if (!slots) {
        memset(g_slot, 0, g_cap * sizeof(uint64_t));
        return 0;
    }
    for (uint32_t i = 0; i < n; ++i) {
        if (slots[i] >= g_cap) return 5;
        g_slot[slots[i]] = 0;
    }
    return 0;
}

/* vocab_size is the vocabulary (out holds n * vocab_size floats), as in the v2 ABI
 * (src/domain/backend_ffi.rs:148-162); slots must be distinct. */
int32_t redukt_backend_forward_batch(uint32_t n, const uint32_t* slots, const uint32_t* toks, float* out,
                                     uint32_t vocab_size) {
    if (vocab_size != g_vocab || n > g_cap) return 5;
    for (uint32_t i = 0; i < n; ++i) {
        if (slots[i] >= g_cap || toks[i] >= g_vocab) return 5;
        for (uint32_t j = 0; j < i; ++j)
            if (slots[j] == slots[i]) return 5;
    }
    if (fail_now()) return 2;
    for (uint32_t i = 0; i < n; ++i) {
        g_slot[slots[i]] = step(g_slot[slots[i]], toks[i]);
        logits_of(g_slot[slots[i]], out + (size_t)i * g_vocab);
    }
    return 0;
}

#ifdef FAKE_PLUGIN_CDF
int32_t redukt_cdf_from_logits(const float* logits, uint32_t n, uint32_t* cdf);
uint32_t redukt_cdf_lookup(const uint32_t* cdf, uint32_t n, uint32_t cum_freq);

/* One step of the n streams, then each row's CDF (n x (vocab + 1) u32 into cdf). */
static int32_t step_cdf(uint32_t n, const uint32_t* slots, const uint32_t* toks, uint32_t* cdf) {
    if (n > g_cap || (n && (!slots || !toks))) return 5;
    for (uint32_t i = 0; i < n; ++i) {
        if (slots[i] >= g_cap || toks[i] >= g_vocab) return 5;
        for (uint32_t j = 0; j < i; ++j)
            if (slots[j] == slots[i]) return 5;
    }
    if (fail_now()) return 2;
    float* lg = (float*)malloc(sizeof(float) * g_vocab);
    if (!lg) return 2;
    for (uint32_t i = 0; i < n; ++i) {
        g_slot[slots[i]] = step(g_slot[slots[i]], toks[i]);
        logits_of(g_slot[slots[i]], lg);
        if (redukt_cdf_from_logits(lg, g_vocab, cdf + (size_t)i * (g_vocab + 1)) != 0) {
            free(lg);
            return 2;
        }
    }
    free(lg);
    return 0;
}

int32_t redukt_backend_forward_batch_cdf(uint32_t n, const uint32_t* slots, const uint32_t* toks, uint32_t* out,
                                         uint32_t cdf_len) {
    if (cdf_len != g_vocab + 1 || !out) return 5;
    return step_cdf(n, slots, toks, out);
}

/* The three values per stream the coder reads for sym[i] (3 u32 a stream into out). */
static int32_t step_sym(uint32_t n, const uint32_t* slots, const uint32_t* toks, const uint32_t* syms,
                        uint32_t* out) {
    for (uint32_t i = 0; i < n; ++i)
        if (syms[i] >= g_vocab) return 5;
    uint32_t* cdf = (uint32_t*)malloc(sizeof(uint32_t) * ((size_t)n * (g_vocab + 1) + 1));
    if (!cdf) return 2;
    const int32_t rc = step_cdf(n, slots, toks, cdf);
    for (uint32_t i = 0; rc == 0 && i < n; ++i) {
        const uint32_t* row = cdf + (size_t)i * (g_vocab + 1);
        out[3 * i] = row[syms[i]];
        out[3 * i + 1] = row[syms[i] + 1];
        out[3 * i + 2] = row[g_vocab];
    }
    free(cdf);
    return rc;
}

int32_t redukt_backend_forward_batch_cdf_sym(uint32_t n, const uint32_t* slots, const uint32_t* toks,
                                             const uint32_t* syms, uint32_t* out, uint32_t vocab) {
    if (vocab != g_vocab || (n && (!syms || !out))) return 5;
    return step_sym(n, slots, toks, syms, out);
}

int32_t redukt_backend_forward_batch_cdf_find(uint32_t n, const uint32_t* slots, const uint32_t* toks,
                                              const uint32_t* targets, uint32_t* out, uint32_t vocab) {
    if (vocab != g_vocab || (n && (!targets || !out))) return 5;
    uint32_t* cdf = (uint32_t*)malloc(sizeof(uint32_t) * ((size_t)n * (g_vocab + 1) + 1));
    if (!cdf) return 2;
    const int32_t rc = step_cdf(n, slots, toks, cdf);
    for (uint32_t i = 0; rc == 0 && i < n; ++i) {
        const uint32_t* row = cdf + (size_t)i * (g_vocab + 1);
        const uint32_t s = redukt_cdf_lookup(row, g_vocab, targets[i]);
        out[4 * i] = s;
        out[4 * i + 1] = s < g_vocab ? row[s] : row[g_vocab];
        out[4 * i + 2] = s < g_vocab ? row[s + 1] : row[g_vocab];
        out[4 * i + 3] = row[g_vocab];
    }
    free(cdf);
    return rc;
}

static struct {
    uint64_t ticket;
    uint32_t n;
    uint32_t* res;
} g_q[2];
static uint64_t g_next_ticket = 1;

static void free_queued(void) {
    for (int k = 0; k < 2; ++k) {
        free(g_q[k].res);
        g_q[k].res = NULL;
        g_q[k].ticket = 0;
    }
}

int32_t redukt_backend_forward_batch_cdf_sym_submit(uint32_t n, const uint32_t* slots, const uint32_t* toks,
                                                    const uint32_t* syms, uint32_t vocab, uint64_t* ticket) {
    if (vocab != g_vocab || !ticket || (n && !syms)) return 5;
    int k = g_q[0].ticket == 0 ? 0 : g_q[1].ticket == 0 ? 1 : -1;
    if (k < 0) return 5;
    uint32_t* res = (uint32_t*)malloc(sizeof(uint32_t) * (3 * (size_t)n + 1));
    if (!res) return 2;
    const int32_t rc = step_sym(n, slots, toks, syms, res);
    if (rc != 0) {
        free(res);
        return rc;
    }
    g_q[k].ticket = g_next_ticket++;
    g_q[k].n = n;
    g_q[k].res = res;
    *ticket = g_q[k].ticket;
    return 0;
}

int32_t redukt_backend_forward_batch_cdf_sym_wait(uint64_t ticket, uint32_t* out, uint32_t n) {
    for (int k = 0; k < 2; ++k) {
        if (ticket == 0 || g_q[k].ticket != ticket) continue;
        if (n != g_q[k].n || (n && !out)) return 5;
        memcpy(out, g_q[k].res, sizeof(uint32_t) * 3 * (size_t)n);
        free(g_q[k].res);
        g_q[k].ticket = 0;
        g_q[k].res = NULL;
        return 0;
    }
    return 5;
}
#else
static void free_queued(void) {}
#endif
