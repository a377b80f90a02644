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

// ------------------------------------------------------------------ random
// The reference's per-thread generator (src/rdv/shaders/libraries/random_library.h,
// after GPU Gems 3 ch. 37: three Tausworthe steps combined with an LCG), restated
// bit for bit so that a dispatch with the same seeds draws the same numbers:
// a thread's state is spawned from the dispatch's uvec4 seeds and its index
// (random_library.h:50-55, 255-267), random() steps the state and maps the
// xor of its words to [0, 1) through the mantissa bits (random_library.h:31-38).
struct RngState {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ uint32_t taus_step(uint32_t z, int s1, int s2, int s3, uint32_t m) {
  const uint32_t b = ((z << s1) ^ z) >> s2;
  return ((z & m) << s3) ^ b;
}

__device__ __forceinline__ void rng_step(RngState& s) {
  s.x = taus_step(s.x, 13, 19, 12, 4294967294u);
  s.y = taus_step(s.y, 2, 25, 4, 4294967288u);
  s.z = taus_step(s.z, 3, 11, 17, 4294967280u);
  s.w = 1664525u * s.w + 1013904223u;
}

__device__ __forceinline__ RngState rng_spawn(const uint32_t (&seeds)[4], int index) {
  const uint32_t i = uint32_t(index);
  RngState s;
  s.x = seeds[0] ^ (i ^ 17u);
  s.y = seeds[1] ^ (i * 123111171u);
  s.z = seeds[2] ^ (i + 11u);
  s.w = seeds[3] ^ (i ^ (seeds[0] + 13u * seeds[1]));
  rng_step(s);
  return s;
}

__device__ __forceinline__ float rng_uniform(RngState& s) {
  rng_step(s);
  const uint32_t v = s.x ^ s.y ^ s.z ^ s.w;
  return __builtin_bit_cast(float, (v & 0x007FFFFFu) | 0x3F800000u) - 1.0f;
}

}  // namespace rdv
