/* The CPU oracle (oracle/liboracle.so) behind the reference's backend plugin ABI
 * (src/domain/backend_ffi.rs:27-177): v1 (init, forward, reset_state, free), v2 (batch_init,
 * batch_reset, forward_batch) and this library's init_ex.  Test infrastructure only: the
 * cross-device round-trip tests code an archive on the CPU through it and decode it on the
 * GPU (and the reverse) with the same lockstep driver.  It serves Mamba .rbin files and
 * RWKV-7 files ("RGPU" version 3, model 2), told apart by the header as the GPU library
 * tells them.  The profile word is the GPU library's (the quantisation bits, bit 5 W8A8,
 * bit 7 for numeric contract 2); the oracle ignores bit 6.
 * v1 and v2 keep disjoint state, as PLUGIN-FFI-V2.md:80-81 requires: two oracle models.
 * Build it with -Wl,-z,nodelete: the oracle's detached worker threads wait inside its code,
 * so it must stay mapped when a driver closes the plugin (a reloaded copy would share the
 * futex addresses of the old workers with new ones). */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
    uint32_t ffi_version, vocab_size, hidden_dim;
    uint8_t name[64];
} BackendInfo;

enum { OK = 0, INIT_FAILED = 1, FORWARD_FAILED = 2, WEIGHTS_NOT_FOUND = 4, INVALID_ARGUMENT = 5 };

/* One oracle model of either kind. */
typedef struct {
    OrcMamba* mamba;
    OrcRwkv* rwkv;
} Model;

static Model g_v1, g_batch;
static char* g_path;
static int g_profile, g_rwkv;
static uint32_t g_vocab, g_hidden;

static int is_rwkv(const char* path) {
    uint32_t h[3] = {0, 0, 0};
    FILE* f = fopen(path, "rb");
    if (!f) return 0;
    const int got = fread(h, 4, 3, f) == 3;
    fclose(f);
    return got && h[0] == 0x55504752u && h[1] == 3 && h[2] == 2;
}

static void model_free(Model* m) {
    if (m->mamba) orc_mamba_free(m->mamba);
    if (m->rwkv) orc_rwkv_free(m->rwkv);
    m->mamba = NULL;
    m->rwkv = NULL;
}

static int model_load(Model* m, uint32_t cap) {
    int err = 0;
    if (g_rwkv) {
        m->rwkv = orc_rwkv_load(g_path, g_profile & ~ORC_PROFILE_EXACT);
        return m->rwkv && orc_rwkv_pool_init(m->rwkv, cap) == 0 ? 0 : -1;
    }
    m->mamba = orc_mamba_load(g_path, g_profile, &err);
    return m->mamba && orc_mamba_pool_init(m->mamba, cap) == 0 ? 0 : -1;
}

static int model_forward(Model* m, uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out) {
    if (m->rwkv) return orc_rwkv_forward(m->rwkv, n, slots, tokens, out) == 0 ? OK : INVALID_ARGUMENT;
    const int rc = orc_mamba_forward(m->mamba, n, slots, tokens, out);
    return rc == 0 ? OK : (rc == 5 ? INVALID_ARGUMENT : FORWARD_FAILED);
}

static int model_reset(Model* m, const uint32_t* slots, uint32_t n) {
    return m->rwkv ? orc_rwkv_reset(m->rwkv, slots, n) : orc_mamba_reset(m->mamba, slots, n);
}

static int model_ready(const Model* m) { return m->mamba != NULL || m->rwkv != NULL; }

void redukt_backend_free(void) {
    model_free(&g_v1);
    model_free(&g_batch);
    free(g_path);
    g_path = NULL;
}

int32_t redukt_backend_init_ex(const uint8_t* weights_path, int32_t device_id, uint32_t profile, BackendInfo* info) {
    (void)device_id;
    if (!weights_path || !info) return INIT_FAILED;
    redukt_backend_free();
    const char* p = (const char*)weights_path;
    const size_t len = strlen(p);
    g_path = (char*)malloc(len + 12);
    if (!g_path) return INIT_FAILED;
    strcpy(g_path, p);
    if (len < 5 || strcmp(p + len - 5, ".rbin") != 0) strcat(g_path, "/model.rbin");
    g_profile = (int)profile;
    g_rwkv = is_rwkv(g_path);
    if (model_load(&g_v1, 1) != 0) return model_ready(&g_v1) ? INIT_FAILED : WEIGHTS_NOT_FOUND;
    if (g_rwkv) {
        uint32_t d[11];
        orc_rwkv_dims(g_v1.rwkv, d);
        g_vocab = d[0];
        g_hidden = d[1];
    } else {
        uint32_t d[8];
        orc_mamba_dims(g_v1.mamba, d);
        g_vocab = d[0];
        g_hidden = d[1];
    }
    memset(info, 0, sizeof(*info));
    info->ffi_version = 1;
    info->vocab_size = g_vocab;
    info->hidden_dim = g_hidden;
    memcpy(info->name, "cpu-oracle", 10);
    return OK;
}

int32_t redukt_backend_init(const uint8_t* weights_path, int32_t device_id, BackendInfo* info) {
    return redukt_backend_init_ex(weights_path, device_id, 0, info);
}

int32_t redukt_backend_forward(uint32_t token, float* out, uint32_t vocab) {
    if (!model_ready(&g_v1) || !out || vocab != g_vocab) return FORWARD_FAILED;
    const uint32_t slot = 0;
    return model_forward(&g_v1, 1, &slot, &token, out) == OK ? OK : FORWARD_FAILED;
}

void redukt_backend_reset_state(void) {
    if (model_ready(&g_v1)) model_reset(&g_v1, NULL, 0);
}

uint32_t redukt_backend_abi_version(void) { return 2; }

int32_t redukt_backend_batch_init(uint32_t max_streams) {
    if (!model_ready(&g_v1)) return INIT_FAILED;
    if (max_streams > 4096) return INVALID_ARGUMENT;
    model_free(&g_batch);
    if (max_streams == 0) return OK;
    return model_load(&g_batch, max_streams) == 0 ? OK : INIT_FAILED;
}

int32_t redukt_backend_batch_reset(const uint32_t* slots, uint32_t n) {
    if (!model_ready(&g_batch)) return INIT_FAILED;
    return model_reset(&g_batch, slots, slots ? n : 0) == 0 ? OK : INVALID_ARGUMENT;
}

int32_t redukt_backend_forward_batch(uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out,
                                     uint32_t vocab) {
    if (!model_ready(&g_batch)) return INIT_FAILED;
    if (vocab != g_vocab) return INVALID_ARGUMENT;
    if (n == 0) return OK;
    return model_forward(&g_batch, n, slots, tokens, out);
}
