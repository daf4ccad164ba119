/* A CPU stand-in for a backend plugin, used by the driver tests only: it exports the v1
 * and v2 plugin symbols with a hash-based recurrent "model" whose logits the tests can
 * recompute in numpy.  State per stream: a u64 s, zero after a reset; a token t moves
 * it to mix(s * 0x100000001b3 + t + 1); the logits of state s are
 *   l[v] = float((mix(s ^ v * 0x9e3779b97f4a7c15) >> 40) % 4001) / 400 - 5    (f32 ops).
 * The weights file holds the vocabulary size as one little-endian u32.
 * FAKE_PLUGIN_ABI=1 in the environment makes abi_version() report a v1-only plugin.
 * FAKE_PLUGIN_FAIL_AFTER=k makes every forward / forward_batch after the first k
 * (counted since init) fail with FORWARD_FAILED. */
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

void redukt_backend_free(void) {
    free(g_slot);
    g_slot = NULL;
    g_cap = 0;
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
