// rwkv_common.h — device helpers shared by the RWKV-7 step kernels (rwkv_step.hip and the
// W8A8 tier, rwkv_a8.hip).
#pragma once
// No a*b+c in this file may be fused: the element-wise arithmetic follows the
// reference operation by operation (a header is compiled before its includer's pragmas).
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>

#include "portable_math.h"

namespace rdk {
namespace {

enum { ACT_NONE = 0, ACT_TANH = 1, ACT_SIGMOID = 2, ACT_RELU2 = 3 };

// tanh_inplace / sigmoid_inplace (tensor.rs:1007-1038) on element r of a length-`len`
// vector: lane form on the 8-aligned body, portable form on the tail; squared_relu_into
// (tensor.rs:1386-1388).
__device__ __forceinline__ float activate(int act, float v, int r, int len) {
    const bool body = r < len / 8 * 8;
    if (act == ACT_TANH)
        return body ? lane_sigmoid_f(v * 2.0f) * 2.0f - 1.0f : 2.0f * (1.0f / (1.0f + exp_f(-(2.0f * v)))) - 1.0f;
    if (act == ACT_SIGMOID) return body ? lane_sigmoid_f(v) : 1.0f / (1.0f + exp_f(-v));
    if (act == ACT_RELU2) {
        const float r2 = v > 0.0f ? v : 0.0f;  // f32::max(v, 0): NaN -> 0
        return r2 * r2;
    }
    return v;
}

}  // namespace
}  // namespace rdk
