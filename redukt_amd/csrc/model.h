// model.h — device-side model and state-pool layout shared by the host code and the
// kernel launchers of libredukt_gpu.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rdk {

// A projection matrix resident in HBM.  Rows are grouped in quads and columns in
// quads; one 4x4 tile (4 rows x 4 consecutive columns) is contiguous: 64 bytes for
// F32, 16 bytes for Q8.  Element (r, k) lives at tile (r/4)*(cols/4) + k/4, offset
// (r%4)*4 + k%4.  A wavefront lane then streams whole tiles with one 16-byte (Q8) or
// four 16-byte (F32) loads and applies each activation quad to four rows at once.
// Rows are zero-padded to a multiple of 4.
struct DMat {
    int rows = 0, cols = 0, rq = 0;  // rq = row quads
    int group = 0;                   // 0: F32; otherwise Q8 columns per scale
    void* w = nullptr;               // tiles
    float* scales = nullptr;         // Q8: [rq*4][cols/group]
    size_t bytes() const;            // HBM bytes of weights + scales
};

struct DLayer {
    float* norm_w = nullptr;
    float* norm_b = nullptr;         // LayerNorm bias (flags bit 0) or null
    DMat in_proj, x_proj, out_proj;
    float* conv_w = nullptr;         // [di][dc]
    float* conv_b = nullptr;         // [di]
    // dt_proj stored transposed, [dr][di], so lane j of a wave reads column j
    // coalesced; F32 in dt_wt, or Q8 in dt_qt with dt_scales[di][dr/dt_group].
    float* dt_wt = nullptr;
    int8_t* dt_qt = nullptr;
    float* dt_scales = nullptr;
    int dt_group = 0;
    float* dt_b = nullptr;           // [di]
    float* a_exp = nullptr;          // [di][16]: exp(A_log), constant per load
    float* d_vec = nullptr;          // [di]
};

struct Dims {
    uint32_t vocab = 0, d = 0, di = 0, ds = 0, dc = 0, dr = 0, nl = 0, flags = 0, tokenizer = 0;
    uint32_t xr() const { return dr + 2 * ds; }
};

// Recurrent state of `cap` slots plus the per-step scratch of `cap` batch rows.
// State layout: conv [layer][slot][di][dc-1] and ssm [layer][slot][di][16], so a
// layer's state for one slot is one contiguous run (18 KB + 96 KB at Mamba-130M).
struct Pool {
    uint32_t cap = 0;
    float* conv = nullptr;
    float* ssm = nullptr;
    float* x = nullptr;        // [cap][d] residual stream
    float* normed = nullptr;   // [cap][d]
    float* xz = nullptr;       // [cap][2*di]
    float* conv_out = nullptr; // [cap][di]
    float* zp = nullptr;       // [cap][xr]
    float* gated = nullptr;    // [cap][di]
    float* out = nullptr;      // [cap][vocab] logits or probabilities
    uint32_t* d_slots = nullptr;
    uint32_t* d_tokens = nullptr;
    uint32_t* h_slots = nullptr;   // pinned staging
    uint32_t* h_tokens = nullptr;
    uint8_t* seen = nullptr;       // host duplicate check, cap bytes
};

// Kernel classes a caller can time with HIP events (see Probe).
enum KernelClass : uint32_t {
    KC_NONE = 0, KC_EMBED = 1, KC_NORM = 2, KC_IN_PROJ = 3, KC_CONV = 4, KC_X_PROJ = 5,
    KC_SCAN = 6, KC_OUT_PROJ = 7, KC_HEAD = 8, KC_SOFTMAX = 9, KC_COUNT = 10
};

// Measurement hook: while cls != KC_NONE, every launch of that class is bracketed by
// two events taken in order from ev[0..cap) (ev is caller-owned); `used` counts them.
struct Probe {
    uint32_t cls = KC_NONE;
    hipEvent_t* ev = nullptr;
    uint32_t cap = 0, used = 0;
};

// Sticky device-side error word for forward_batch_device (bit 0: bad slot or token,
// bit 1: duplicate slot).
struct StepArgs {
    const Dims* dims;
    const DLayer* layers;
    const DMat* emb;
    const DMat* head;
    const float* norm_f_w;
    const float* norm_f_b;
    Pool* pool;
    uint32_t n;
    const uint32_t* slots;   // device
    const uint32_t* tokens;  // device
    float* out;              // device [n][vocab]
    bool probs;
    bool check;              // run the device-side argument check
    uint32_t* err;           // device error word
    Probe* probe;            // may be null
};

// Enqueue one full step on `stream`.  Returns hipSuccess or the first launch error.
hipError_t enqueue_step(const StepArgs& a, hipStream_t stream);
// Zero the state of the n slots listed in d_slots (device).
hipError_t enqueue_reset(const Dims& dims, Pool& pool, const uint32_t* d_slots, uint32_t n, hipStream_t stream);

}  // namespace rdk
