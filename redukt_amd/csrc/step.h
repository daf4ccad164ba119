// step.h — a step as a list of kernel launches (issued directly or recorded as a graph).
#pragma once
// No a*b+c in this file may be fused: the element-wise arithmetic follows the
// reference operation by operation (a header is compiled before its includer's pragmas).
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstring>
#include <memory>

namespace rdk {

struct Launch {
    const void* fn;
    dim3 grid, block;
    uint32_t lds;
    uint32_t cls;
    bool coop = false;   // cooperative launch (every workgroup resident at once); never captured
    std::unique_ptr<unsigned char[]> args;
    void* argp;
    template <typename A>
    static Launch make(const void* fn, dim3 g, dim3 b, uint32_t lds, uint32_t cls, const A& a) {
        Launch l;
        l.fn = fn;
        l.grid = g;
        l.block = b;
        l.lds = lds;
        l.cls = cls;
        l.args.reset(new unsigned char[sizeof(A)]);
        memcpy(l.args.get(), &a, sizeof(A));
        l.argp = l.args.get();
        return l;
    }
};

struct TMat;
struct Pool;
struct StepIO;

// Launches shared by the step builders of both models (kernels in mamba_step.hip).
// embed: x = emb[token] with the device argument check; with xw, the pre-staged
// activations of the first RMSNorm consumer.  head: ws selects the weights-stationary
// head (Q8 per-row, activations pre-staged in xw; ssp null = already normed); otherwise
// the streamed head norms x itself (LayerNorm when nb is given, RMSNorm otherwise, or
// pre-staged xw/ssp).
Launch embed_launch(const TMat& emb, Pool& p, const StepIO& io, const float* nw0, __bf16* xw, float* ssp, int ks_x,
                    int tiles);
Launch head_launch(const TMat& H, Pool& p, const StepIO& io, const float* x, const float* nw, const float* nb,
                   const __bf16* xw, const float* ssp, int d, int tiles, bool ws);
Launch softmax_launch(float* out, int vocab, uint32_t n);
// The scan of one layer over n streams of pool p (its x_proj partials, u, z and slots),
// writing the gated vector as bf16 limb tiles (glimb) or as f32 rows (g32).
struct DLayer;
struct Dims;
Launch scan_launch(const DLayer& L, const Dims& D, Pool& p, uint32_t n, bool exact, __bf16* glimb, float* g32,
                   float* ssm_layer);
// The scan of the reference-order tier: the complete x_proj outputs of each stream in
// xpart (one block), the portable exp, the dt_proj dot in numeric contract 1 or (fma) 2,
// the gated vector as f32 rows.
Launch scan_exact_launch(const DLayer& L, const Dims& D, Pool& p, uint32_t n, bool fma, float* g32, float* ssm_layer);
// The wavefront-GEMV tier: whether a chunks-per-lane count is compiled.
bool gemv_cpl_supported(int cpl);
// Logits [rows][n] -> CDF [rows][n + 1] on the device, bit for bit the host coding path's
// cdf_from_logits (cdf_step.hip); `scratch` holds cdf_scratch_bytes(rows, n).
size_t cdf_scratch_bytes(uint32_t rows, uint32_t n);
hipError_t cdf_launch(const float* logits, uint32_t rows, uint32_t n, void* scratch, uint32_t* cdf, hipStream_t st);
// out[3r .. 3r + 2] = cdf[r][sym[r]], cdf[r][sym[r] + 1], cdf[r][n] for rows r (cdf rows of n + 1).
hipError_t cdf_pick_launch(const uint32_t* cdf, uint32_t rows, uint32_t n, const uint32_t* sym, uint32_t* out,
                           hipStream_t st);
// The decoder's symbol for each row's target cumulative frequency, with its two bounds and
// the row's total (4 u32 a row).
hipError_t cdf_find_launch(const uint32_t* cdf, uint32_t rows, uint32_t n, const uint32_t* cum, uint32_t* out,
                           hipStream_t st);

namespace {

template <typename K>
void allow_lds(K* fn, uint32_t bytes) {
    static uint32_t set = 0;
    if (bytes > set) {
        (void)hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
        set = bytes;
    }
}

}  // namespace
}  // namespace rdk
