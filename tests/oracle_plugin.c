/* The CPU oracle (oracle/liboracle.so) behind the reference's backend plugin ABI
 * (src/domain/backend_ffi.rs:27-177): v1 (init, forward, reset_state, free), v2 (batch_init,
 * batch_reset, forward_batch) and this library's init_ex.  Test infrastructure only: the
 * cross-device round-trip tests code an archive on the CPU through it and decode it on the
 * GPU (and the reverse) with the same lockstep driver.  The profile word is the GPU
 * library's (the quantisation bits, bit 7 for numeric contract 2); the oracle ignores bit 6.
 * v1 and v2 keep disjoint state, as PLUGIN-FFI-V2.md:80-81 requires: two oracle models.
 * Build it with -Wl,-z,nodelete: the oracle's detached worker threads wait inside its code,
 * so it must stay mapped when a driver closes the plugin (a reloaded copy would share the
 * futex addresses of the old workers with new ones). */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

typedef struct {
    uint32_t ffi_version, vocab_size, hidden_dim;
    uint8_t name[64];
} BackendInfo;

enum { OK = 0, INIT_FAILED = 1, FORWARD_FAILED = 2, WEIGHTS_NOT_FOUND = 4, INVALID_ARGUMENT = 5 };

static OrcMamba* g_v1;
static OrcMamba* g_batch;
static char* g_path;
static int g_profile;
static uint32_t g_vocab;

void redukt_backend_free(void) {
    if (g_v1) orc_mamba_free(g_v1);
    if (g_batch) orc_mamba_free(g_batch);
    g_v1 = g_batch = NULL;
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
    int err = 0;
    g_v1 = orc_mamba_load(g_path, g_profile, &err);
    if (!g_v1) return WEIGHTS_NOT_FOUND;
    if (orc_mamba_pool_init(g_v1, 1) != 0) return INIT_FAILED;
    uint32_t d[8];
    orc_mamba_dims(g_v1, d);
    g_vocab = d[0];
    memset(info, 0, sizeof(*info));
    info->ffi_version = 1;
    info->vocab_size = d[0];
    info->hidden_dim = d[1];
    memcpy(info->name, "cpu-oracle", 10);
    return OK;
}

int32_t redukt_backend_init(const uint8_t* weights_path, int32_t device_id, BackendInfo* info) {
    return redukt_backend_init_ex(weights_path, device_id, 0, info);
}

int32_t redukt_backend_forward(uint32_t token, float* out, uint32_t vocab) {
    if (!g_v1 || !out || vocab != g_vocab) return FORWARD_FAILED;
    const uint32_t slot = 0;
    return orc_mamba_forward(g_v1, 1, &slot, &token, out) == 0 ? OK : FORWARD_FAILED;
}

void redukt_backend_reset_state(void) {
    if (g_v1) orc_mamba_reset(g_v1, NULL, 0);
}

uint32_t redukt_backend_abi_version(void) { return 2; }

int32_t redukt_backend_batch_init(uint32_t max_streams) {
    if (!g_v1) return INIT_FAILED;
    if (max_streams > 4096) return INVALID_ARGUMENT;
    if (g_batch) orc_mamba_free(g_batch);
    g_batch = NULL;
    if (max_streams == 0) return OK;
    int err = 0;
    g_batch = orc_mamba_load(g_path, g_profile, &err);
    if (!g_batch || orc_mamba_pool_init(g_batch, max_streams) != 0) return INIT_FAILED;
    return OK;
}

int32_t redukt_backend_batch_reset(const uint32_t* slots, uint32_t n) {
    if (!g_batch) return INIT_FAILED;
    return orc_mamba_reset(g_batch, slots, slots ? n : 0) == 0 ? OK : INVALID_ARGUMENT;
}

int32_t redukt_backend_forward_batch(uint32_t n, const uint32_t* slots, const uint32_t* tokens, float* out,
                                     uint32_t vocab) {
    if (!g_batch) return INIT_FAILED;
    if (vocab != g_vocab) return INVALID_ARGUMENT;
    if (n == 0) return OK;
    const int rc = orc_mamba_forward(g_batch, n, slots, tokens, out);
    return rc == 0 ? OK : (rc == 5 ? INVALID_ARGUMENT : FORWARD_FAILED);
}
