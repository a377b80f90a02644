// C ABI entry points: host-side validation, error reporting and kernel dispatch.
#include <mutex>
#include <string>

#include "mlp_layout.h"
#include "rdv_common.h"

namespace rdv {

// ------------------------------------------------------------------ errors
static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(RDV_ERR_HIP, std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")");
}

// ------------------------------------------------------------ device info
int device_info(DeviceInfo* out) {
  static std::mutex mu;
  static DeviceInfo cache[64];
  static bool have[64] = {};
  int dev = 0;
  RDV_HIP_TRY(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) return fail(RDV_ERR_UNSUPPORTED, "device index out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!have[dev]) {
    int cus = 0, lds = 0;
    RDV_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    RDV_HIP_TRY(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev));
    cache[dev].cu_count = cus;
    cache[dev].lds_per_block = size_t(lds);
    have[dev] = true;
  }
  *out = cache[dev];
  return RDV_OK;
}

// ---------------------------------------------------------- MLP launchers
struct FusedEntry;
const FusedEntry* find_fused(const rdv_mlp_desc& d, const MlpLayout& lay);
const char* fused_name(const FusedEntry* e);
int launch_fused_entry(const FusedEntry* e, const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                       const float* x, float* y, int64_t nrows, hipStream_t stream);
bool generic_f16_supported(const rdv_mlp_desc& d);
const char* generic_f16_name(const rdv_mlp_desc& d, const MlpLayout& lay);
int launch_mlp_generic_f16(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* x, float* y,
                           int64_t nrows, hipStream_t stream);
int launch_mlp_chain_f32(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* x,
                         float* y, int64_t row0, int64_t nrows, bool force_f32, hipStream_t stream,
                         const DirectWeights* dw = nullptr);
int launch_fused_entry_direct(const FusedEntry* e, const rdv_mlp_desc& d, const MlpLayout& lay,
                              const DirectWeights& dw, const float* x, float* y, int64_t nrows, hipStream_t stream);
bool direct_fused_ok(const FusedEntry* e, const rdv_mlp_desc& d);
int launch_mlp_pack(const rdv_mlp_desc& d, const MlpLayout& lay, const float* const* W, const float* const* b,
                    void* packed, hipStream_t stream);
int prepare_chain_f32(const rdv_mlp_desc& d);
const char* chain_f32_name(const rdv_mlp_desc& d, const MlpLayout& lay);
int64_t winograd_weight_bytes(int cin, int cout);
int launch_winograd_transform_weight(const void* w, int w_layout, int w_dtype, int cin, int cout, void* U,
                                     hipStream_t stream);
int train_check(const rdv_mlp_desc& d, const MlpLayout& lay);
int64_t train_workspace_bytes(const rdv_mlp_desc& d, const MlpLayout& lay, int64_t n, int cu);
int launch_train_step(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const void* x,
                      const float* target, int64_t n, void* workspace, int64_t ws_bytes, float* loss,
                      float* const* dW, float* const* db, hipStream_t stream);
int launch_train_step_static(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const void* x,
                             const float* target, int64_t n, float* loss, float* const* dW, float* const* db,
                             hipStream_t stream);
int launch_camera_rays(const rdv_camera_desc& c, const float* poses, const uint32_t* seeds, float* rays,
                       hipStream_t stream);
int launch_cameras_rays_at(const rdv_camera_desc& c, const float* poses, const int32_t* idx, int64_t n,
                           const uint32_t* seeds, float* rays, hipStream_t stream);
int launch_grid_gather(const float* values, int rank, const int64_t* shape, int width, const int32_t* idx, int64_t n,
                       float* out, hipStream_t stream);
int launch_random_uniform(const uint32_t* seeds, int64_t n_threads, int per_thread, float* out, hipStream_t stream);
int launch_ratiotracking(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                         const rdv_ratiotracking_desc& rt, const float* majorant, const float* rays, int64_t nrays,
                         float* out, hipStream_t stream);
int launch_volume_profile(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed,
                          const rdv_volume_profile_desc& vp, const float* majorant, const float* dda_grid, int dda_w,
                          int dda_h, int dda_d, const float* rays, int64_t nrays, float* out, float* spos,
                          float* env_dirs, float* env_w, int32_t* valid, hipStream_t stream);
int launch_volume_profile_finish(const rdv_volume_profile_desc& vp, const float* albedo, int64_t albedo_stride,
                                 const float* env, int64_t env_stride, const float* env_w, const int32_t* valid,
                                 int64_t nrays, float* out, hipStream_t stream);
int launch_broadcast_rows(const float* value, int width, int64_t rows, float* out, hipStream_t stream);
int launch_voxel_majorant(const float* grid, int mw, int mh, int md, const float* rays, int64_t n, float* out,
                          hipStream_t stream);
int launch_majorant_grid(const rdv_majorant_grid_desc& g, const float* fine, float* out, hipStream_t stream);
int launch_render_ea(const rdv_camera_desc& c, const float* poses, const float* rays, int64_t n_rays,
                     const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, int samples, float* image,
                     hipStream_t stream);
int launch_composite(const float* sigma_rgb, const float* dts, int64_t nrays, int samples, float* out,
                     hipStream_t stream);
int launch_raymarch_transmittance(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* rays,
                                  int64_t nrays, const float* transform12, float step, float density_scale,
                                  float* out, hipStream_t stream);
int launch_winograd3x3(const rdv_conv_desc& d, const void* x, const void* U, const float* bias, void* y,
                       hipStream_t stream);

int linear_op_check(const rdv_linear_op_desc& d, std::string* why);
int launch_linear_op(const rdv_linear_op_desc& d, const float* x, const void* w, const float* bias, float* y,
                     hipStream_t stream);
int launch_relu_op(const float* x, float* y, int64_t n, hipStream_t stream);

int conv2d_check(const rdv_conv2d_desc& d, std::string* why);
int launch_conv2d(const rdv_conv2d_desc& d, const float* x, const float* w, const float* bias, float* y,
                  hipStream_t stream);
int launch_downsample2x(const float* x, int64_t H, int64_t W, int C, float* y, hipStream_t stream);
int launch_upsample2x(const float* x, int64_t H, int64_t W, int C, float* y, hipStream_t stream);
int launch_concat(const float* x1, int C1, const float* x2, int C2, int64_t rows, float* y, hipStream_t stream);

static bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

static int check_linear_op(const rdv_linear_op_desc* d) {
  if (!d) return fail(RDV_ERR_INVALID, "linear op descriptor is NULL");
  std::string why;
  if (linear_op_check(*d, &why) != RDV_OK) return fail(RDV_ERR_INVALID, why);
  return RDV_OK;
}

static int check_conv(const rdv_conv_desc* d) {
  if (!d) return fail(RDV_ERR_INVALID, "conv descriptor is NULL");
  if (d->batch < 1) return fail(RDV_ERR_INVALID, "batch must be >= 1");
  if (d->H < 2 || d->W < 2 || d->H % 2 || d->W % 2)
    return fail(RDV_ERR_INVALID, "H (" + std::to_string(d->H) + ") and W (" + std::to_string(d->W) +
                                     ") must be even and >= 2");
  if (d->cin < 1 || d->cin > 64)
    return fail(RDV_ERR_INVALID, "in_channels (" + std::to_string(d->cin) + ") must be in [1, 64]");
  if (d->cout < 16 || d->cout > 1024 || d->cout % 16)
    return fail(RDV_ERR_INVALID, "out_channels (" + std::to_string(d->cout) + ") must be a multiple of 16 in [16, 1024]");
  if ((d->in_layout != RDV_LAYOUT_HWC && d->in_layout != RDV_LAYOUT_CHW) ||
      (d->out_layout != RDV_LAYOUT_HWC && d->out_layout != RDV_LAYOUT_CHW))
    return fail(RDV_ERR_INVALID, "unknown image layout");
  if ((d->in_dtype != RDV_DTYPE_F32 && d->in_dtype != RDV_DTYPE_F16) ||
      (d->out_dtype != RDV_DTYPE_F32 && d->out_dtype != RDV_DTYPE_F16))
    return fail(RDV_ERR_INVALID, "unknown element type");
  // per-image element offsets are 32-bit in the kernel
  if (int64_t(d->H) * d->W * d->cin >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "H * W * in_channels must be < 2^31");
  const int64_t px = int64_t(d->batch) * d->H * d->W;
  if (px > (int64_t(1) << 40)) return fail(RDV_ERR_INVALID, "image too large");
  return RDV_OK;
}

static int check_mlp(const rdv_mlp_desc* d, MlpLayout* lay) {
  if (!d) return fail(RDV_ERR_INVALID, "mlp descriptor is NULL");
  if (d->n_layers < 1 || d->n_layers > RDV_MLP_MAX_LAYERS)
    return fail(RDV_ERR_INVALID, "n_layers must be in [1, " + std::to_string(RDV_MLP_MAX_LAYERS) + "], got " +
                                     std::to_string(d->n_layers));
  if (d->in_features < 1) return fail(RDV_ERR_INVALID, "in_features must be >= 1");
  for (int i = 0; i <= d->n_layers; ++i) {
    if (d->dims[i] < 1 || d->dims[i] > RDV_MLP_MAX_WIDTH)
      return fail(RDV_ERR_INVALID, "dims[" + std::to_string(i) + "] = " + std::to_string(d->dims[i]) +
                                       " outside [1, " + std::to_string(RDV_MLP_MAX_WIDTH) + "]");
  }
  if (d->encoding == RDV_ENC_NONE) {
    if (d->dims[0] != d->in_features)
      return fail(RDV_ERR_INVALID, "weight's in_features (" + std::to_string(d->dims[0]) +
                                       ") must match x's trailing dim (" + std::to_string(d->in_features) + ")");
  } else if (d->encoding == RDV_ENC_FREQ) {
    if (d->enc_octaves < 1 || d->enc_octaves > 16) return fail(RDV_ERR_INVALID, "enc_octaves must be in [1, 16]");
    const int w = d->in_features * (1 + 2 * d->enc_octaves);
    if (d->dims[0] < w)
      return fail(RDV_ERR_INVALID, "layer 0 in_features (" + std::to_string(d->dims[0]) +
                                       ") is smaller than the encoded width (" + std::to_string(w) + ")");
  } else {
    return fail(RDV_ERR_INVALID, "unknown encoding " + std::to_string(d->encoding));
  }
  for (int i = 0; i < d->n_layers; ++i) {
    if (d->act[i] < RDV_ACT_NONE || d->act[i] > RDV_ACT_DENSITY_RGB)
      return fail(RDV_ERR_INVALID, "unknown activation code " + std::to_string(d->act[i]));
    if (d->prec[i] != RDV_PREC_F32 && d->prec[i] != RDV_PREC_F16)
      return fail(RDV_ERR_INVALID, "unknown precision code " + std::to_string(d->prec[i]));
  }
  if (!mlp_layout(*d, lay)) return fail(RDV_ERR_INVALID, "invalid layer chain");
  for (int i = 0; i < d->n_layers; ++i)
    if (lay->kc[i] * 16 > 2 * RDV_MLP_MAX_WIDTH) return fail(RDV_ERR_INVALID, "encoded width too large");
  return RDV_OK;
}

}  // namespace rdv

using namespace rdv;

extern "C" {

const char* rdv_last_error(void) { return g_last_error.c_str(); }

int rdv_version(void) { return 100; }

int rdv_device_cu_count(void) {
  DeviceInfo di;
  if (device_info(&di) != RDV_OK) return 0;
  return di.cu_count;
}

int rdv_mlp_validate(const rdv_mlp_desc* desc) {
  MlpLayout lay;
  return check_mlp(desc, &lay);
}

int64_t rdv_mlp_packed_bytes(const rdv_mlp_desc* desc) {
  MlpLayout lay;
  const int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  return lay.total_bytes;
}

int rdv_mlp_pack(const rdv_mlp_desc* desc, const float* const* weights, const float* const* biases, void* packed,
                 void* stream) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  if (!weights || !biases || !packed) return fail(RDV_ERR_INVALID, "rdv_mlp_pack: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(packed) % 256 != 0)
    return fail(RDV_ERR_INVALID, "rdv_mlp_pack: packed buffer must be 256-byte aligned");
  for (int i = 0; i < desc->n_layers; ++i)
    if (!weights[i] || !biases[i])
      return fail(RDV_ERR_INVALID, "rdv_mlp_pack: NULL weight or bias of layer " + std::to_string(i));
  return launch_mlp_pack(*desc, lay, weights, biases, packed, static_cast<hipStream_t>(stream));
}

static int mlp_forward_impl(const rdv_mlp_desc* desc, const void* packed, const float* x, float* y, int64_t n,
                            void* stream, bool tail_f32) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  if (n < 0) return fail(RDV_ERR_INVALID, "row count must be >= 0");
  if (n == 0) return RDV_OK;
  if (!packed || !x || !y) return fail(RDV_ERR_INVALID, "rdv_mlp_forward: NULL pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t n_full = tail_f32 ? (n / 32) * 32 : n;
  const int64_t n_tail = n - n_full;
  const FusedEntry* e = find_fused(*desc, lay);
  if (e) {
    rc = launch_fused_entry(e, *desc, lay, packed, x, y, n_full, s);
  } else if (generic_f16_supported(*desc)) {
    rc = launch_mlp_generic_f16(*desc, lay, packed, x, y, n_full, s);
  } else {
    rc = prepare_chain_f32(*desc);
    if (rc == RDV_OK) rc = launch_mlp_chain_f32(*desc, lay, packed, x, y, 0, n_full, false, s);
  }
  if (rc != RDV_OK) return rc;
  if (n_tail > 0) {
    rc = prepare_chain_f32(*desc);
    if (rc == RDV_OK) rc = launch_mlp_chain_f32(*desc, lay, packed, x, y, n_full, n_tail, true, s);
  }
  return rc;
}

int rdv_mlp_forward(const rdv_mlp_desc* desc, const void* packed, const float* x, float* y, int64_t n,
                    void* stream) {
  return mlp_forward_impl(desc, packed, x, y, n, stream, true);
}

int64_t rdv_mlp_unpacked_workspace_bytes(const rdv_mlp_desc* desc) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  if (direct_fused_ok(find_fused(*desc, lay), *desc)) return 0;
  return lay.total_bytes;
}

int rdv_mlp_forward_unpacked(const rdv_mlp_desc* desc, const float* const* weights, const float* const* biases,
                             const float* x, float* y, int64_t n, void* workspace, int64_t workspace_bytes,
                             void* stream) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  if (n < 0) return fail(RDV_ERR_INVALID, "row count must be >= 0");
  if (!weights || !biases) return fail(RDV_ERR_INVALID, "rdv_mlp_forward_unpacked: NULL parameter array");
  DirectWeights dw = {};
  for (int i = 0; i < desc->n_layers; ++i) {
    if (!weights[i] || !biases[i]) return fail(RDV_ERR_INVALID, "rdv_mlp_forward_unpacked: NULL layer parameter");
    dw.W[i] = weights[i];
    dw.b[i] = biases[i];
  }
  if (n == 0) return RDV_OK;
  if (!x || !y) return fail(RDV_ERR_INVALID, "rdv_mlp_forward_unpacked: NULL pointer argument");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const FusedEntry* e = find_fused(*desc, lay);
  if (!direct_fused_ok(e, *desc)) {  // pack into the workspace, then the packed path
    if (workspace_bytes < lay.total_bytes || workspace == nullptr)
      return fail(RDV_ERR_WORKSPACE, "workspace of " + std::to_string(workspace_bytes) + " bytes; this chain needs " +
                                         std::to_string(lay.total_bytes));
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return fail(RDV_ERR_INVALID, "workspace must be 256-byte aligned");
    rc = launch_mlp_pack(*desc, lay, dw.W, dw.b, workspace, s);
    if (rc != RDV_OK) return rc;
    return mlp_forward_impl(desc, workspace, x, y, n, stream, true);
  }
  const int64_t n_full = (n / 32) * 32;
  rc = launch_fused_entry_direct(e, *desc, lay, dw, x, y, n_full, s);
  if (rc != RDV_OK) return rc;
  if (n > n_full) {
    rc = prepare_chain_f32(*desc);
    if (rc == RDV_OK) rc = launch_mlp_chain_f32(*desc, lay, nullptr, x, y, n_full, n - n_full, true, s, &dw);
  }
  return rc;
}

int rdv_mlp_forward_f16_all(const rdv_mlp_desc* desc, const void* packed, const float* x, float* y, int64_t n,
                            void* stream) {
  return mlp_forward_impl(desc, packed, x, y, n, stream, false);
}

int rdv_winograd3x3_validate(const rdv_conv_desc* desc) { return check_conv(desc); }

int64_t rdv_winograd3x3_weight_bytes(int32_t cin, int32_t cout) {
  if (cin < 1 || cin > 64 || cout < 16 || cout > 1024 || cout % 16)
    return fail(RDV_ERR_INVALID, "in_channels must be in [1, 64], out_channels a multiple of 16 in [16, 1024]");
  return winograd_weight_bytes(cin, cout);
}

int rdv_winograd3x3_transform_weight(const void* w, int32_t w_layout, int32_t w_dtype, int32_t cin, int32_t cout,
                                     void* U, void* stream) {
  const int64_t nb = rdv_winograd3x3_weight_bytes(cin, cout);
  if (nb < 0) return int(nb);
  if (!w || !U) return fail(RDV_ERR_INVALID, "rdv_winograd3x3_transform_weight: NULL pointer argument");
  if (w_layout != RDV_WLAYOUT_RSCK && w_layout != RDV_WLAYOUT_KCRS) return fail(RDV_ERR_INVALID, "unknown filter layout");
  if (w_dtype != RDV_DTYPE_F32 && w_dtype != RDV_DTYPE_F16) return fail(RDV_ERR_INVALID, "unknown filter type");
  if (reinterpret_cast<uintptr_t>(U) % 16) return fail(RDV_ERR_INVALID, "U must be 16-byte aligned");
  return launch_winograd_transform_weight(w, w_layout, w_dtype, cin, cout, U, static_cast<hipStream_t>(stream));
}

int rdv_winograd3x3_forward(const rdv_conv_desc* desc, const void* x, const void* U, const float* bias, void* y,
                            void* stream) {
  int rc = check_conv(desc);
  if (rc != RDV_OK) return rc;
  if (!x || !U || !y) return fail(RDV_ERR_INVALID, "rdv_winograd3x3_forward: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(U) % 16) return fail(RDV_ERR_INVALID, "U must be 16-byte aligned");
  const size_t oal = desc->out_dtype == RDV_DTYPE_F16 ? 8 : 16;
  if (reinterpret_cast<uintptr_t>(y) % oal) return fail(RDV_ERR_INVALID, "y is not aligned for vector stores");
  return launch_winograd3x3(*desc, x, U, bias, y, static_cast<hipStream_t>(stream));
}

int rdv_linear_op_validate(const rdv_linear_op_desc* desc) { return check_linear_op(desc); }

int rdv_linear_op(const rdv_linear_op_desc* desc, const float* x, const void* weight, const float* bias, float* y,
                  void* stream) {
  if (int rc = check_linear_op(desc)) return rc;
  if (desc->rows == 0) return RDV_OK;
  if (!x || !weight || !bias || !y) return fail(RDV_ERR_INVALID, "linear op: NULL pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(RDV_ERR_INVALID, "linear op: x and y must be 16-byte aligned");
  if (desc->wkind != RDV_WKIND_F16_TILED16 && !aligned16(weight))
    return fail(RDV_ERR_INVALID, "linear op: weight must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(weight) & 1) != 0) return fail(RDV_ERR_INVALID, "linear op: weight misaligned");
  if ((reinterpret_cast<uintptr_t>(bias) & 3) != 0) return fail(RDV_ERR_INVALID, "linear op: bias misaligned");
  return launch_linear_op(*desc, x, weight, bias, y, static_cast<hipStream_t>(stream));
}

int rdv_relu_op(const float* x, float* y, int64_t n, void* stream) {
  if (n < 0) return fail(RDV_ERR_INVALID, "relu op: n must be >= 0");
  if (n == 0) return RDV_OK;
  if (!x || !y) return fail(RDV_ERR_INVALID, "relu op: NULL pointer");
  if (!aligned16(x) || !aligned16(y)) return fail(RDV_ERR_INVALID, "relu op: x and y must be 16-byte aligned");
  return launch_relu_op(x, y, n, static_cast<hipStream_t>(stream));
}

static int check_conv2d(const rdv_conv2d_desc* d) {
  if (!d) return fail(RDV_ERR_INVALID, "conv2d descriptor is NULL");
  std::string why;
  if (conv2d_check(*d, &why) != RDV_OK) return fail(RDV_ERR_INVALID, "conv2d: " + why);
  return RDV_OK;
}

int rdv_conv2d_validate(const rdv_conv2d_desc* desc) { return check_conv2d(desc); }

int rdv_conv2d(const rdv_conv2d_desc* desc, const float* x, const float* w, const float* bias, float* y,
               void* stream) {
  if (int rc = check_conv2d(desc)) return rc;
  if (int64_t(desc->H) * desc->W == 0) return RDV_OK;
  if (!x || !w || !y) return fail(RDV_ERR_INVALID, "conv2d: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(x) % 4 || reinterpret_cast<uintptr_t>(y) % 4)
    return fail(RDV_ERR_INVALID, "conv2d: x and y must be 4-byte aligned");
  if (reinterpret_cast<uintptr_t>(w) % 4 || reinterpret_cast<uintptr_t>(bias) % 4)
    return fail(RDV_ERR_INVALID, "conv2d: w and bias must be 4-byte aligned");
  return launch_conv2d(*desc, x, w, bias, y, static_cast<hipStream_t>(stream));
}

static int check_image(const char* what, int64_t H, int64_t W, int32_t C) {
  if (H < 0 || W < 0) return fail(RDV_ERR_INVALID, std::string(what) + ": H and W must be >= 0");
  if (C < 1) return fail(RDV_ERR_INVALID, std::string(what) + ": channels (" + std::to_string(C) + ") must be >= 1");
  if (H > (int64_t(1) << 24) || W > (int64_t(1) << 24) || H * W > (int64_t(1) << 40) / C)
    return fail(RDV_ERR_INVALID, std::string(what) + ": image too large");
  return RDV_OK;
}

int rdv_downsample2x(const float* x, int64_t H, int64_t W, int32_t C, float* y, void* stream) {
  if (int rc = check_image("downsample2x", H, W, C)) return rc;
  if (H % 2 || W % 2) return fail(RDV_ERR_INVALID, "downsample2x: H and W must be even");
  if (H == 0 || W == 0) return RDV_OK;
  if (!x || !y) return fail(RDV_ERR_INVALID, "downsample2x: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(x) % 4 || reinterpret_cast<uintptr_t>(y) % 4)
    return fail(RDV_ERR_INVALID, "downsample2x: x and y must be 4-byte aligned");
  return launch_downsample2x(x, H, W, C, y, static_cast<hipStream_t>(stream));
}

int rdv_upsample2x(const float* x, int64_t H, int64_t W, int32_t C, float* y, void* stream) {
  if (int rc = check_image("upsample2x", H, W, C)) return rc;
  if (H == 0 || W == 0) return RDV_OK;
  if (!x || !y) return fail(RDV_ERR_INVALID, "upsample2x: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(x) % 4 || reinterpret_cast<uintptr_t>(y) % 4)
    return fail(RDV_ERR_INVALID, "upsample2x: x and y must be 4-byte aligned");
  return launch_upsample2x(x, H, W, C, y, static_cast<hipStream_t>(stream));
}

int rdv_concat_channels(const float* x1, int32_t C1, const float* x2, int32_t C2, int64_t rows, float* y,
                        void* stream) {
  if (C1 < 4 || C1 % 4 || C2 < 4 || C2 % 4)
    return fail(RDV_ERR_INVALID, "concat: channel counts must be positive multiples of 4");
  if (rows < 0 || rows > (int64_t(1) << 40) / (int64_t(C1) + C2)) return fail(RDV_ERR_INVALID, "concat: bad row count");
  if (rows == 0) return RDV_OK;
  if (!x1 || !x2 || !y) return fail(RDV_ERR_INVALID, "concat: NULL pointer argument");
  if (!aligned16(x1) || !aligned16(x2) || !aligned16(y))
    return fail(RDV_ERR_INVALID, "concat: x1, x2 and y must be 16-byte aligned");
  return launch_concat(x1, C1, x2, C2, rows, y, static_cast<hipStream_t>(stream));
}

int64_t rdv_mlp_train_workspace_bytes(const rdv_mlp_desc* desc, int64_t n) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  rc = train_check(*desc, lay);
  if (rc != RDV_OK) return rc;
  if (n < 1) return fail(RDV_ERR_INVALID, "n must be >= 1");
  DeviceInfo di;
  rc = device_info(&di);
  if (rc != RDV_OK) return rc;
  return train_workspace_bytes(*desc, lay, n, di.cu_count);
}

int rdv_mlp_train_step(const rdv_mlp_desc* desc, const void* packed, const void* x, const float* target, int64_t n,
                       void* workspace, int64_t workspace_bytes, float* loss, float* const* dW, float* const* db,
                       void* stream) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  rc = train_check(*desc, lay);
  if (rc != RDV_OK) return rc;
  if (n < 1) return fail(RDV_ERR_INVALID, "n must be >= 1");
  if (!packed || !x || !target || !workspace || !loss || !dW || !db)
    return fail(RDV_ERR_INVALID, "rdv_mlp_train_step: NULL pointer argument");
  for (int i = 0; i < desc->n_layers; ++i)
    if (!dW[i] || !db[i]) return fail(RDV_ERR_INVALID, "rdv_mlp_train_step: NULL gradient pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(target) % 16 ||
      reinterpret_cast<uintptr_t>(workspace) % 256)
    return fail(RDV_ERR_INVALID, "x and target must be 16-byte aligned, the workspace 256-byte aligned");
  return launch_train_step(*desc, lay, packed, x, target, n, workspace, workspace_bytes, loss, dW, db,
                           static_cast<hipStream_t>(stream));
}

int rdv_mlp_train_step_static(const rdv_mlp_desc* desc, const void* packed, const void* x, const float* target,
                              int64_t n, float* loss, float* const* dW, float* const* db, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(desc, &lay);
  if (rc != RDV_OK) return rc;
  rc = train_check(*desc, lay);
  if (rc != RDV_OK) return rc;
  if (n < 1) return fail(RDV_ERR_INVALID, "n must be >= 1");
  if (!packed || !x || !target || !loss || !dW || !db)
    return fail(RDV_ERR_INVALID, "rdv_mlp_train_step_static: NULL pointer argument");
  for (int i = 0; i < desc->n_layers; ++i)
    if (!dW[i] || !db[i]) return fail(RDV_ERR_INVALID, "rdv_mlp_train_step_static: NULL gradient pointer");
  if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(target) % 16)
    return fail(RDV_ERR_INVALID, "x and target must be 16-byte aligned");
  return launch_train_step_static(*desc, lay, packed, x, target, n, loss, dW, db, static_cast<hipStream_t>(stream));
}

static int check_camera(const rdv_camera_desc* c) {
  if (!c) return fail(RDV_ERR_INVALID, "camera descriptor is NULL");
  if (c->n_cams < 1 || c->width < 1 || c->height < 1)
    return fail(RDV_ERR_INVALID, "cameras need n_cams, width and height >= 1");
  if (int64_t(c->n_cams) * c->width * c->height > (int64_t(1) << 40)) return fail(RDV_ERR_INVALID, "too many rays");
  if (!(c->fov > 0.0f && c->fov < 3.14159265f)) return fail(RDV_ERR_INVALID, "fov must be in (0, pi)");
  if (!(c->aspect_ratio > 0.0f)) return fail(RDV_ERR_INVALID, "aspect_ratio must be > 0");
  return RDV_OK;
}

int rdv_cameras_rays(const rdv_camera_desc* cam, const float* poses, float* rays, void* stream) {
  int rc = check_camera(cam);
  if (rc != RDV_OK) return rc;
  if (!poses || !rays) return fail(RDV_ERR_INVALID, "rdv_cameras_rays: NULL pointer argument");
  return launch_camera_rays(*cam, poses, nullptr, rays, static_cast<hipStream_t>(stream));
}

int rdv_cameras_rays_jittered(const rdv_camera_desc* cam, const float* poses, const uint32_t* seeds, float* rays,
                              void* stream) {
  int rc = check_camera(cam);
  if (rc != RDV_OK) return rc;
  if (!poses || !rays || !seeds) return fail(RDV_ERR_INVALID, "rdv_cameras_rays_jittered: NULL pointer argument");
  if (int64_t(cam->n_cams) * cam->height * cam->width >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "a jittered dispatch holds fewer than 2^31 cells (the generator's thread index is an int)");
  return launch_camera_rays(*cam, poses, seeds, rays, static_cast<hipStream_t>(stream));
}

int rdv_cameras_rays_at(const rdv_camera_desc* cam, const float* poses, const int32_t* indices, int64_t n,
                        const uint32_t* seeds, float* rays, void* stream) {
  int rc = check_camera(cam);
  if (rc != RDV_OK) return rc;
  if (n < 0 || n >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "the batch holds fewer than 2^31 index vectors (the generator's thread index is an int)");
  if (n == 0) return RDV_OK;
  if (!poses || !indices || !rays) return fail(RDV_ERR_INVALID, "rdv_cameras_rays_at: NULL pointer argument");
  return launch_cameras_rays_at(*cam, poses, indices, n, seeds, rays, static_cast<hipStream_t>(stream));
}

int rdv_grid_gather(const float* values, int32_t rank, const int64_t* shape, int32_t width, const int32_t* indices,
                    int64_t n, float* out, void* stream) {
  if (rank < 1 || rank > RDV_GRID_MAX_RANK)
    return fail(RDV_ERR_INVALID, "grid rank must be in [1, " + std::to_string(RDV_GRID_MAX_RANK) + "], got " +
                                     std::to_string(rank));
  if (!shape) return fail(RDV_ERR_INVALID, "rdv_grid_gather: NULL shape");
  int64_t cells = 1;
  for (int d = 0; d < rank; ++d) {
    if (shape[d] < 1) return fail(RDV_ERR_INVALID, "grid dimensions must be >= 1");
    if (cells > (int64_t(1) << 40) / shape[d]) return fail(RDV_ERR_INVALID, "grid too large");
    cells *= shape[d];
  }
  if (width < 1) return fail(RDV_ERR_INVALID, "width must be >= 1");
  if (n < 0 || n > ((int64_t(1) << 40) / width)) return fail(RDV_ERR_INVALID, "batch size out of range");
  if (n == 0) return RDV_OK;
  if (!values || !indices || !out) return fail(RDV_ERR_INVALID, "rdv_grid_gather: NULL pointer argument");
  return launch_grid_gather(values, rank, shape, width, indices, n, out, static_cast<hipStream_t>(stream));
}

int rdv_random_uniform(const uint32_t* seeds, int64_t n_threads, int32_t per_thread, float* out, void* stream) {
  if (n_threads < 0 || n_threads >= (int64_t(1) << 31)) return fail(RDV_ERR_INVALID, "n_threads must be in [0, 2^31)");
  if (per_thread < 0 || per_thread > (1 << 20)) return fail(RDV_ERR_INVALID, "per_thread must be in [0, 2^20]");
  if (n_threads == 0 || per_thread == 0) return RDV_OK;
  if (!seeds || !out) return fail(RDV_ERR_INVALID, "rdv_random_uniform: NULL pointer argument");
  return launch_random_uniform(seeds, n_threads, per_thread, out, static_cast<hipStream_t>(stream));
}

int rdv_render_emission_absorption(const rdv_camera_desc* cam, const float* poses, const rdv_mlp_desc* field,
                                   const void* packed, int32_t samples, float* image, void* stream) {
  int rc = check_camera(cam);
  if (rc != RDV_OK) return rc;
  MlpLayout lay;
  rc = check_mlp(field, &lay);
  if (rc != RDV_OK) return rc;
  if (samples < 32 || samples % 32 || samples > (1 << 20))
    return fail(RDV_ERR_INVALID, "samples must be a positive multiple of 32 (at most 2^20)");
  if (!poses || !packed || !image) return fail(RDV_ERR_INVALID, "rdv_render_emission_absorption: NULL pointer argument");
  return launch_render_ea(*cam, poses, nullptr, 0, *field, lay, packed, samples, image,
                          static_cast<hipStream_t>(stream));
}

int rdv_render_emission_absorption_rays(const rdv_mlp_desc* field, const void* packed, const float* rays,
                                        int64_t n_rays, int32_t samples, float* out, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(field, &lay);
  if (rc != RDV_OK) return rc;
  if (samples < 32 || samples % 32 || samples > (1 << 20))
    return fail(RDV_ERR_INVALID, "samples must be a positive multiple of 32 (at most 2^20)");
  if (n_rays < 0 || n_rays > (int64_t(1) << 40)) return fail(RDV_ERR_INVALID, "bad ray count");
  if (n_rays == 0) return RDV_OK;
  if (!packed || !rays || !out) return fail(RDV_ERR_INVALID, "rdv_render_emission_absorption_rays: NULL pointer argument");
  const rdv_camera_desc none{1, 1, 1, 1.0f, 1.0f};
  return launch_render_ea(none, nullptr, rays, n_rays, *field, lay, packed, samples, out,
                          static_cast<hipStream_t>(stream));
}

int rdv_composite(const float* sigma_rgb, const float* dt, int64_t n_rays, int32_t samples, float* out,
                  void* stream) {
  if (n_rays < 0 || samples < 1) return fail(RDV_ERR_INVALID, "rdv_composite: n_rays >= 0 and samples >= 1 required");
  if (n_rays == 0) return RDV_OK;
  if (!sigma_rgb || !dt || !out) return fail(RDV_ERR_INVALID, "rdv_composite: NULL pointer argument");
  if (reinterpret_cast<uintptr_t>(sigma_rgb) % 16) return fail(RDV_ERR_INVALID, "sigma_rgb must be 16-byte aligned");
  return launch_composite(sigma_rgb, dt, n_rays, samples, out, static_cast<hipStream_t>(stream));
}

int rdv_raymarch_transmittance(const rdv_mlp_desc* extinction, const void* packed, const float* rays,
                               int64_t n_rays, const float* transform12, float step_size, float density_scale,
                               float* out, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(extinction, &lay);
  if (rc != RDV_OK) return rc;
  if (n_rays < 0) return fail(RDV_ERR_INVALID, "n_rays must be >= 0");
  if (!(step_size > 0.0f)) return fail(RDV_ERR_INVALID, "step_size must be > 0");
  if (!transform12) return fail(RDV_ERR_INVALID, "transform is NULL");
  if (n_rays == 0) return RDV_OK;
  if (!packed || !rays || !out) return fail(RDV_ERR_INVALID, "rdv_raymarch_transmittance: NULL pointer argument");
  return launch_raymarch_transmittance(*extinction, lay, packed, rays, n_rays, transform12, step_size, density_scale,
                                       out, static_cast<hipStream_t>(stream));
}

int rdv_ratiotracking_transmittance(const rdv_mlp_desc* extinction, const void* packed,
                                    const rdv_ratiotracking_desc* rt, const float* majorant, const float* rays,
                                    int64_t n_rays, float* out, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(extinction, &lay);
  if (rc != RDV_OK) return rc;
  if (!rt) return fail(RDV_ERR_INVALID, "rdv_ratiotracking_transmittance: NULL descriptor");
  if (n_rays < 0 || n_rays >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "n_rays must be in [0, 2^31) (the generator's thread index is an int)");
  if (rt->maj_width < 1 || rt->maj_height < 1 || rt->maj_depth < 1 ||
      int64_t(rt->maj_width) * rt->maj_height * rt->maj_depth >= (int64_t(1) << 40))
    return fail(RDV_ERR_INVALID, "the majorant grid needs width, height, depth >= 1");
  if (!(rt->density_scale > 0.0f)) return fail(RDV_ERR_INVALID, "density_scale must be > 0");
  if (rt->rng_skip < 0 || rt->rng_skip > 1024) return fail(RDV_ERR_INVALID, "rng_skip must be in [0, 1024]");
  if (rt->reserved != 0) return fail(RDV_ERR_INVALID, "reserved must be 0");
  if (n_rays == 0) return RDV_OK;
  if (!packed || !majorant || !rays || !out)
    return fail(RDV_ERR_INVALID, "rdv_ratiotracking_transmittance: NULL pointer argument");
  return launch_ratiotracking(*extinction, lay, packed, *rt, majorant, rays, n_rays, out,
                              static_cast<hipStream_t>(stream));
}

static int check_volume_profile(const rdv_volume_profile_desc* vp) {
  if (!vp) return fail(RDV_ERR_INVALID, "volume profile: NULL descriptor");
  if (vp->depth_samples < 1 || vp->depth_samples > RDV_VP_MAX_DEPTH)
    return fail(RDV_ERR_INVALID, "depth_samples must be in [1, " + std::to_string(RDV_VP_MAX_DEPTH) + "]");
  if (vp->spectral_dim < 1 || vp->spectral_dim > RDV_VP_MAX_SPECTRAL)
    return fail(RDV_ERR_INVALID, "spectral_dim must be in [1, " + std::to_string(RDV_VP_MAX_SPECTRAL) + "]");
  if (vp->sample_index < 0 || vp->sample_index >= vp->depth_samples)
    return fail(RDV_ERR_INVALID, "sample_index must index one of the depth samples");
  if (vp->environment_samples < 0 || vp->environment_samples > 4096)
    return fail(RDV_ERR_INVALID, "environment_samples must be in [0, 4096]");
  if (!(vp->step_size > 0.0f)) return fail(RDV_ERR_INVALID, "step_size must be > 0");
  if (!(vp->density_scale > 0.0f)) return fail(RDV_ERR_INVALID, "density_scale must be > 0");
  if (vp->maj_width < 1 || vp->maj_height < 1 || vp->maj_depth < 1 ||
      int64_t(vp->maj_width) * vp->maj_height * vp->maj_depth >= (int64_t(1) << 40))
    return fail(RDV_ERR_INVALID, "the majorant grid needs width, height, depth >= 1");
  if (vp->rng_skip < 0 || vp->rng_skip > 1024) return fail(RDV_ERR_INVALID, "rng_skip must be in [0, 1024]");
  if (vp->reserved != 0) return fail(RDV_ERR_INVALID, "reserved must be 0");
  return RDV_OK;
}

int rdv_volume_profile(const rdv_mlp_desc* extinction, const void* packed, const rdv_volume_profile_desc* vp,
                       const float* majorant, const float* rays, int64_t n_rays, float* out, float* sample_pos,
                       float* env_dirs, float* env_weights, int32_t* valid, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(extinction, &lay);
  if (rc != RDV_OK) return rc;
  rc = check_volume_profile(vp);
  if (rc != RDV_OK) return rc;
  if (n_rays < 0 || n_rays >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "n_rays must be in [0, 2^31) (the generator's thread index is an int)");
  if (n_rays == 0) return RDV_OK;
  if (!packed || !majorant || !rays || !out || !sample_pos || !valid ||
      (vp->environment_samples > 0 && (!env_dirs || !env_weights)))
    return fail(RDV_ERR_INVALID, "rdv_volume_profile: NULL pointer argument");
  return launch_volume_profile(*extinction, lay, packed, *vp, majorant, nullptr, 0, 0, 0, rays, n_rays, out,
                               sample_pos, env_dirs, env_weights, valid, static_cast<hipStream_t>(stream));
}

int rdv_volume_profile_dda(const rdv_mlp_desc* extinction, const void* packed, const rdv_volume_profile_desc* vp,
                           const float* majorant, const float* majorant_grid, int32_t grid_width,
                           int32_t grid_height, int32_t grid_depth, const float* rays, int64_t n_rays, float* out,
                           float* sample_pos, float* env_dirs, float* env_weights, int32_t* valid, void* stream) {
  MlpLayout lay;
  int rc = check_mlp(extinction, &lay);
  if (rc != RDV_OK) return rc;
  rc = check_volume_profile(vp);
  if (rc != RDV_OK) return rc;
  if (grid_width < 1 || grid_height < 1 || grid_depth < 1 || grid_width > 4096 || grid_height > 4096 ||
      grid_depth > 4096)
    return fail(RDV_ERR_INVALID, "rdv_volume_profile_dda: grid dimensions must be in [1, 4096]");
  if (n_rays < 0 || n_rays >= (int64_t(1) << 31))
    return fail(RDV_ERR_INVALID, "n_rays must be in [0, 2^31) (the generator's thread index is an int)");
  if (n_rays == 0) return RDV_OK;
  if (!packed || !majorant || !majorant_grid || !rays || !out || !sample_pos || !valid ||
      (vp->environment_samples > 0 && (!env_dirs || !env_weights)))
    return fail(RDV_ERR_INVALID, "rdv_volume_profile_dda: NULL pointer argument");
  return launch_volume_profile(*extinction, lay, packed, *vp, majorant, majorant_grid, grid_width, grid_height,
                               grid_depth, rays, n_rays, out, sample_pos, env_dirs, env_weights, valid,
                               static_cast<hipStream_t>(stream));
}

int rdv_volume_profile_finish(const rdv_volume_profile_desc* vp, const float* albedo, int64_t albedo_stride,
                              const float* env, int64_t env_stride, const float* env_weights,
                              const int32_t* valid, int64_t n_rays, float* out, void* stream) {
  int rc = check_volume_profile(vp);
  if (rc != RDV_OK) return rc;
  if (n_rays < 0) return fail(RDV_ERR_INVALID, "n_rays must be >= 0");
  if (albedo_stride < 0 || env_stride < 0) return fail(RDV_ERR_INVALID, "row strides must be >= 0");
  if (n_rays == 0) return RDV_OK;
  if (!albedo || !valid || !out || (vp->environment_samples > 0 && (!env || !env_weights)))
    return fail(RDV_ERR_INVALID, "rdv_volume_profile_finish: NULL pointer argument");
  return launch_volume_profile_finish(*vp, albedo, albedo_stride, env, env_stride, env_weights, valid, n_rays, out,
                                      static_cast<hipStream_t>(stream));
}

int rdv_broadcast_rows(const float* value, int32_t width, int64_t rows, float* out, void* stream) {
  if (width < 1) return fail(RDV_ERR_INVALID, "width must be >= 1");
  if (rows < 0) return fail(RDV_ERR_INVALID, "rows must be >= 0");
  if (rows == 0) return RDV_OK;
  if (!value || !out) return fail(RDV_ERR_INVALID, "rdv_broadcast_rows: NULL pointer argument");
  return launch_broadcast_rows(value, width, rows, out, static_cast<hipStream_t>(stream));
}

int rdv_voxel_majorant(const float* grid, int32_t width, int32_t height, int32_t depth, const float* rays,
                       int64_t n_rays, float* out, void* stream) {
  if (width < 1 || height < 1 || depth < 1) return fail(RDV_ERR_INVALID, "the grid needs width, height, depth >= 1");
  if (n_rays < 0) return fail(RDV_ERR_INVALID, "n_rays must be >= 0");
  if (n_rays == 0) return RDV_OK;
  if (!grid || !rays || !out) return fail(RDV_ERR_INVALID, "rdv_voxel_majorant: NULL pointer argument");
  return launch_voxel_majorant(grid, width, height, depth, rays, n_rays, out, static_cast<hipStream_t>(stream));
}

int rdv_majorant_grid(const rdv_majorant_grid_desc* desc, const float* fine, float* out, void* stream) {
  if (!desc) return fail(RDV_ERR_INVALID, "rdv_majorant_grid: NULL descriptor");
  if (desc->rank < 1 || desc->rank > 4) return fail(RDV_ERR_INVALID, "rank must be 1..4");
  if (desc->channels < 1) return fail(RDV_ERR_INVALID, "channels must be >= 1");
  int64_t fine_cells = 1, cells = 1;
  for (int d = 0; d < desc->rank; ++d) {
    if (desc->fine_shape[d] < 1 || desc->shape[d] < 1)
      return fail(RDV_ERR_INVALID, "every extent of both shapes must be >= 1");
    fine_cells *= desc->fine_shape[d];
    cells *= desc->shape[d];
    if (fine_cells > (int64_t(1) << 40) || cells > (int64_t(1) << 40)) return fail(RDV_ERR_INVALID, "grid too large");
  }
  if (!fine || !out) return fail(RDV_ERR_INVALID, "rdv_majorant_grid: NULL pointer argument");
  return launch_majorant_grid(*desc, fine, out, static_cast<hipStream_t>(stream));
}

const char* rdv_mlp_kernel_name(const rdv_mlp_desc* desc) {
  MlpLayout lay;
  if (check_mlp(desc, &lay) != RDV_OK) return "";
  const FusedEntry* e = find_fused(*desc, lay);
  if (e) return fused_name(e);
  return generic_f16_supported(*desc) ? generic_f16_name(*desc, lay) : chain_f32_name(*desc, lay);
}

}  // extern "C"
