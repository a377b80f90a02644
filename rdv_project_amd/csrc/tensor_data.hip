// Data-movement tensor operations over channels-last fp32 images [H*W, C]:
// 2x2 average-pool downsample, nearest-neighbour 2x upsample and channel concat.
//
// Replace the reference's Downsample2xTensorOp / Upsample2xTensorOp /
// ConcatTensorOp dispatches (src/rdv/domain/nn.py:1090-1150,
// src/rdv/shaders/tensors/{downsample2x,upsample2x,concat}_tensor_op.h), which
// assign one 4-row x 8-channel tile per thread.  Here each lane moves one
// 16-byte group of 4 channels, so a wave reads and writes contiguous 1 KiB
// spans of a row (whole 128-byte lines per instruction); a grid-stride loop
// covers the image.  HBM-bound: the minimum traffic is each input and output
// byte once.  The arithmetic is the reference's: the downsample sums its four
// taps left to right in fp32, ((x00 + x01) + x10) + x11, then scales by 0.25.
#include "rdv_common.h"

namespace rdv {

namespace {

// I: the index type, 32-bit whenever every index fits (its divisions are
// several times cheaper than 64-bit ones, and these kernels have only a few
// VALU operations per 16 bytes to spend).
template <typename I>
__global__ __launch_bounds__(256) void downsample2x_kernel(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                           I Wo, I c4, I total) {
  const I stride = I(gridDim.x) * blockDim.x;
  const I row_in = 2 * Wo * c4;  // one input image row, in 16-byte groups
  for (I i = I(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I c = i % c4, pix = i / c4;
    const I oh = pix / Wo, ow = pix % Wo;
    const I base = (2 * oh) * row_in + (2 * ow) * c4 + c;
    const f32x4 a = x[base], b = x[base + c4], d0 = x[base + row_in], d1 = x[base + row_in + c4];
    f32x4 v;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = (((a[j] + b[j]) + d0[j]) + d1[j]) * 0.25f;
    __builtin_nontemporal_store(v, y + i);
  }
}

template <typename I>
__global__ __launch_bounds__(256) void upsample2x_kernel(const f32x4* __restrict__ x, f32x4* __restrict__ y,
                                                         I Wo, I c4, I total) {
  const I stride = I(gridDim.x) * blockDim.x;
  const I Wi = Wo / 2;
  for (I i = I(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I c = i % c4, pix = i / c4;
    const I oh = pix / Wo, ow = pix % Wo;
    __builtin_nontemporal_store(x[((oh / 2) * Wi + ow / 2) * c4 + c], y + i);
  }
}

template <typename I>
__global__ __launch_bounds__(256) void concat_kernel(const f32x4* __restrict__ x1, const f32x4* __restrict__ x2,
                                                     f32x4* __restrict__ y, I c4a, I c4b, I total) {
  const I stride = I(gridDim.x) * blockDim.x;
  const I c4 = c4a + c4b;
  for (I i = I(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I c = i % c4, row = i / c4;
    const f32x4 v = c < c4a ? x1[row * c4a + c] : x2[row * c4b + (c - c4a)];
    __builtin_nontemporal_store(v, y + i);
  }
}

// Per-element versions for channel counts that are not a multiple of 4 (or
// buffers that are not 16-byte aligned): the same arithmetic, one float per lane.
__global__ __launch_bounds__(256) void downsample2x_scalar_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                  int64_t Wo, int64_t C, int64_t total) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t row_in = 2 * Wo * C;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % C, pix = i / C;
    const int64_t oh = pix / Wo, ow = pix % Wo;
    const int64_t base = (2 * oh) * row_in + (2 * ow) * C + c;
    y[i] = (((x[base] + x[base + C]) + x[base + row_in]) + x[base + row_in + C]) * 0.25f;
  }
}

__global__ __launch_bounds__(256) void upsample2x_scalar_kernel(const float* __restrict__ x, float* __restrict__ y,
                                                                int64_t Wo, int64_t C, int64_t total) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  const int64_t Wi = Wo / 2;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t c = i % C, pix = i / C;
    const int64_t oh = pix / Wo, ow = pix % Wo;
    y[i] = x[((oh / 2) * Wi + ow / 2) * C + c];
  }
}

bool vec_ok(const void* a, const void* b, int C) {
  return C % 4 == 0 && reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(b) % 16 == 0;
}

// Every index of a launch (input and output, plus a grid-stride step past the
// end) below 2^32?
bool fits32(int64_t in_groups, int64_t out_groups) {
  const int64_t lim = (int64_t(1) << 32) - (int64_t(1) << 26);
  return in_groups < lim && out_groups < lim;
}

int grid_for(int64_t total, unsigned* blocks) {
  DeviceInfo di;
  const int rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  int64_t b = (total + 255) / 256;
  const int64_t cap = int64_t(di.cu_count) * 16;
  *blocks = unsigned(b < cap ? (b < 1 ? 1 : b) : cap);
  return RDV_OK;
}

}  // namespace

int launch_downsample2x(const float* x, int64_t H, int64_t W, int C, float* y, hipStream_t stream) {
  if (!vec_ok(x, y, C)) {
    const int64_t n = (H / 2) * (W / 2) * C;
    if (n == 0) return RDV_OK;
    unsigned blocks = 0;
    if (int rc = grid_for(n, &blocks)) return rc;
    downsample2x_scalar_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(x, y, W / 2, C, n);
    RDV_HIP_TRY(hipGetLastError());
    return RDV_OK;
  }
  const int64_t total = (H / 2) * (W / 2) * (C / 4);
  if (total == 0) return RDV_OK;
  unsigned blocks = 0;
  if (int rc = grid_for(total, &blocks)) return rc;
  const f32x4* xs = reinterpret_cast<const f32x4*>(x);
  f32x4* ys = reinterpret_cast<f32x4*>(y);
  if (fits32(H * W * (C / 4), total))
    downsample2x_kernel<uint32_t><<<dim3(blocks), dim3(256), 0, stream>>>(xs, ys, uint32_t(W / 2), uint32_t(C / 4),
                                                                         uint32_t(total));
  else
    downsample2x_kernel<int64_t><<<dim3(blocks), dim3(256), 0, stream>>>(xs, ys, W / 2, int64_t(C / 4), total);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_upsample2x(const float* x, int64_t H, int64_t W, int C, float* y, hipStream_t stream) {
  if (!vec_ok(x, y, C)) {
    const int64_t n = (2 * H) * (2 * W) * C;
    if (n == 0) return RDV_OK;
    unsigned blocks = 0;
    if (int rc = grid_for(n, &blocks)) return rc;
    upsample2x_scalar_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(x, y, 2 * W, C, n);
    RDV_HIP_TRY(hipGetLastError());
    return RDV_OK;
  }
  const int64_t total = (2 * H) * (2 * W) * (C / 4);
  if (total == 0) return RDV_OK;
  unsigned blocks = 0;
  if (int rc = grid_for(total, &blocks)) return rc;
  const f32x4* xs = reinterpret_cast<const f32x4*>(x);
  f32x4* ys = reinterpret_cast<f32x4*>(y);
  if (fits32(H * W * (C / 4), total))
    upsample2x_kernel<uint32_t><<<dim3(blocks), dim3(256), 0, stream>>>(xs, ys, uint32_t(2 * W), uint32_t(C / 4),
                                                                       uint32_t(total));
  else
    upsample2x_kernel<int64_t><<<dim3(blocks), dim3(256), 0, stream>>>(xs, ys, 2 * W, int64_t(C / 4), total);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

int launch_concat(const float* x1, int C1, const float* x2, int C2, int64_t rows, float* y, hipStream_t stream) {
  const int64_t total = rows * ((C1 + C2) / 4);
  if (total == 0) return RDV_OK;
  unsigned blocks = 0;
  if (int rc = grid_for(total, &blocks)) return rc;
  const f32x4* a = reinterpret_cast<const f32x4*>(x1);
  const f32x4* b = reinterpret_cast<const f32x4*>(x2);
  f32x4* ys = reinterpret_cast<f32x4*>(y);
  if (fits32(total, total))
    concat_kernel<uint32_t><<<dim3(blocks), dim3(256), 0, stream>>>(a, b, ys, uint32_t(C1 / 4), uint32_t(C2 / 4),
                                                                   uint32_t(total));
  else
    concat_kernel<int64_t><<<dim3(blocks), dim3(256), 0, stream>>>(a, b, ys, int64_t(C1 / 4), int64_t(C2 / 4), total);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

// Constant map over rows (src/rdv/maths/__init__.py:1659-1668): out[r, c] = value[c].
__global__ __launch_bounds__(256) void broadcast_rows_kernel(const float* __restrict__ value, int width, int64_t total,
                                                             float* __restrict__ out) {
  for (int64_t e = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += int64_t(gridDim.x) * blockDim.x)
    out[e] = value[e % width];
}

int launch_broadcast_rows(const float* value, int width, int64_t rows, float* out, hipStream_t stream) {
  const int64_t total = rows * width;
  unsigned blocks = 0;
  if (int rc = grid_for(total, &blocks)) return rc;
  broadcast_rows_kernel<<<dim3(blocks), dim3(256), 0, stream>>>(value, width, total, out);
  RDV_HIP_TRY(hipGetLastError());
  return RDV_OK;
}

}  // namespace rdv
