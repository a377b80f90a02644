// Shared types and helpers for the gfx950 kernels and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/rdv_hip.h"

namespace rdv {

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef half_t half2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- errors
// Thread-local message of the last failure; set by fail(), read by rdv_last_error().
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

#define RDV_HIP_TRY(expr)                                    \
  do {                                                       \
    hipError_t _e = (expr);                                  \
    if (_e != hipSuccess) return ::rdv::hip_fail(_e, #expr); \
  } while (0)

// Device properties of the current device, cached per device index.
struct DeviceInfo {
  int cu_count;
  size_t lds_per_block;
};
int device_info(DeviceInfo* out);

// ----------------------------------------------------------- activations
// Shared by every kernel that applies an activation so that all paths agree.
__device__ __forceinline__ float softplus_f(float x) {
  // log(1 + exp(x)) = max(x, 0) + log1p(exp(-|x|)), stable for any x.
  return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x)));
}
__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

// Hardware-instruction versions (v_exp_f32 / v_log_f32 / v_rcp_f32, ~1 ulp each)
// for heads inside matrix-core kernels.
__device__ __forceinline__ float fast_softplus(float x) {
  // max(x, 0) + ln(1 + 2^(-|x| log2 e)); the argument of the log is in [1, 2]
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  return fmaxf(x, 0.0f) + __builtin_amdgcn_logf(1.0f + e) * 0.6931471805599453f;
}
__device__ __forceinline__ float fast_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

__device__ __forceinline__ float apply_act(int act, int channel, float v) {
  switch (act) {
    case RDV_ACT_RELU: return fmaxf(v, 0.0f);
    case RDV_ACT_SOFTPLUS: return softplus_f(v);
    case RDV_ACT_SIGMOID: return sigmoid_f(v);
    case RDV_ACT_DENSITY_RGB: return channel == 0 ? softplus_f(v) : sigmoid_f(v);
    default: return v;
  }
}

}  // namespace rdv
