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
int launch_mlp_chain_f32(const rdv_mlp_desc& d, const MlpLayout& lay, const void* packed, const float* x,
                         float* y, int64_t row0, int64_t nrows, bool force_f32, hipStream_t stream);
int launch_mlp_pack(const rdv_mlp_desc& d, const MlpLayout& lay, const float* const* W, const float* const* b,
                    void* packed, hipStream_t stream);
int prepare_chain_f32(const rdv_mlp_desc& d);

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

int rdv_mlp_forward_f16_all(const rdv_mlp_desc* desc, const void* packed, const float* x, float* y, int64_t n,
                            void* stream) {
  return mlp_forward_impl(desc, packed, x, y, n, stream, false);
}

const char* rdv_mlp_kernel_name(const rdv_mlp_desc* desc) {
  MlpLayout lay;
  if (check_mlp(desc, &lay) != RDV_OK) return "";
  const FusedEntry* e = find_fused(*desc, lay);
  return e ? fused_name(e) : "mlp_chain_f32_kernel";
}

}  // extern "C"
