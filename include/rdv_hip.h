/*
 * rdv_hip.h — C ABI of the MI355X (gfx950) small-network hot path.
 *
 * The reference (rendervous/rdv_project) has no native FFI: every hot-path
 * kernel there is a GLSL snippet stitched into one compute shader and submitted
 * through `dispatch()` (src/rdv/core/_core.py:2799-2886).  Each entry point below
 * replaces one such dispatch for one node family; the comment on each names the
 * reference node and shader it stands in for.  The Python package
 * `rdv_project_amd` binds these with ctypes (see rdv_project_amd/_lib.py).
 *
 * Conventions
 *  - Every tensor argument is a caller-owned DEVICE pointer (e.g. a torch
 *    tensor's data_ptr()).  Nothing on a forward path allocates device memory;
 *    scratch, where a kernel needs it, is passed in by the caller.
 *  - `stream` is a hipStream_t (NULL = the legacy default stream).  Launches are
 *    stream-ordered and asynchronous; the caller synchronises if it needs to.
 *  - Every function returns RDV_OK (0) or a negative rdv_status.  The message of
 *    the last failure on the calling thread is returned by rdv_last_error().
 *  - Shapes are validated on the host before anything is launched, so a bad
 *    descriptor is an error code, never a GPU fault (the reference's equivalent
 *    checks are host asserts, e.g. src/rdv/domain/nn.py:37-39, 1064-1078).
 */
#ifndef RDV_HIP_H
#define RDV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ status */
typedef enum rdv_status {
  RDV_OK = 0,
  RDV_ERR_INVALID = -1,     /* bad descriptor / shape / pointer (reference: AssertionError) */
  RDV_ERR_UNSUPPORTED = -2, /* valid request this build does not implement               */
  RDV_ERR_HIP = -3,         /* a HIP runtime call failed                                  */
  RDV_ERR_WORKSPACE = -4    /* caller-provided workspace too small                        */
} rdv_status;

/* Message of the last failing call on this thread ("" if none). */
const char* rdv_last_error(void);
/* ABI version of this library (major * 100 + minor). */
int rdv_version(void);
/* Number of compute units of the current device (0 if no device). */
int rdv_device_cu_count(void);

/* --------------------------------------------------------------- fused MLP */
#define RDV_MLP_MAX_LAYERS 16
#define RDV_MLP_MAX_WIDTH 256

/* Activation applied to a layer's output. RELU is the reference's ReLU map
 * (src/rdv/shaders/maps/relu.h:1-5); the others are build-defined heads for
 * the emission-absorption renderer (no counterpart in the reference). */
enum {
  RDV_ACT_NONE = 0,
  RDV_ACT_RELU = 1,
  RDV_ACT_SOFTPLUS = 2,   /* log(1 + exp(x))                                   */
  RDV_ACT_SIGMOID = 3,    /* 1 / (1 + exp(-x))                                 */
  RDV_ACT_DENSITY_RGB = 4 /* channel 0 softplus, channels 1.. sigmoid          */
};

/* Arithmetic of a layer.
 * F16: LinearFast (src/rdv/shaders/maps/linear_fast.h:39-100): input and weight
 *      rounded to fp16, products accumulated in fp32, fp32 bias added after.
 * F32: Linear (src/rdv/shaders/maps/linear.h:15-44): exact fp32,
 *      acc = bias; acc += x[k] * W[o][k] for k ascending. */
enum { RDV_PREC_F32 = 0, RDV_PREC_F16 = 1 };

/* Input encoding applied to each row of x before layer 0 (build-defined; the
 * reference has no encoding node).  FREQ with L octaves maps p[0..D) to
 *   [p_0..p_{D-1}, for k in 0..L-1: sin(2^k pi p_0..D-1), cos(2^k pi p_0..D-1)]
 * followed by zeros up to enc_width. */
enum { RDV_ENC_NONE = 0, RDV_ENC_FREQ = 1 };

typedef struct rdv_mlp_desc {
  int32_t n_layers;                       /* 1..RDV_MLP_MAX_LAYERS                     */
  int32_t in_features;                    /* width of each row of x                    */
  int32_t encoding;                       /* RDV_ENC_*                                 */
  int32_t enc_octaves;                    /* FREQ: number of octaves L                 */
  int32_t dims[RDV_MLP_MAX_LAYERS + 1];   /* dims[0] = layer-0 input width (= encoded  */
                                          /* width), dims[i+1] = output width of i     */
  int32_t act[RDV_MLP_MAX_LAYERS];        /* RDV_ACT_* after layer i                   */
  int32_t prec[RDV_MLP_MAX_LAYERS];       /* RDV_PREC_* of layer i                     */
} rdv_mlp_desc;

/* Host-only shape check of a descriptor; launches nothing. */
int rdv_mlp_validate(const rdv_mlp_desc* desc);

/* Size in bytes of the packed parameter block for `desc` (< 0 on error). */
int64_t rdv_mlp_packed_bytes(const rdv_mlp_desc* desc);

/* Packs the layers' parameters into `packed` (device, rdv_mlp_packed_bytes
 * bytes, 256-byte aligned), every layer and the header in one launch.
 * weights[i] points to layer i's fp32 weight, row-major [dims[i+1], dims[i]]
 * (PyTorch nn.Linear layout), biases[i] to its fp32 bias [dims[i+1]]; both
 * arrays hold DEVICE pointers and live on the host.
 * Replaces the per-node weight/bias upload of _LinearBase.__init__
 * (src/rdv/domain/nn.py:34-54). */
int rdv_mlp_pack(const rdv_mlp_desc* desc, const float* const* weights,
                 const float* const* biases, void* packed, void* stream);

/* y[n, dims[L]] = chain(x[n, in_features]) for fp32 row-major x and y.  Every
 * all-LinearFast chain runs on the fp16 matrix cores (a compile-time kernel for
 * the benchmark shapes, a runtime-shaped one for the rest); chains with an
 * exact fp32 Linear layer run on the vector ALUs.
 * Replaces Map.__call__ -> dispatch(MapEvaluator) over a chain of
 * LinearFast / Linear / ReLU maps (src/rdv/maths/__init__.py:1451-1487,
 * src/rdv/shaders/maps/map_evaluator.h:1-5, composite.h:8-12).
 * Rows are processed in groups of 32 as the reference's workgroups are; when n
 * is not a multiple of 32 the last partial group is evaluated in exact fp32,
 * which is what the reference's LinearFast does for a partial workgroup
 * (linear_fast.h:102-108 behind all_thread_sync,
 * src/rdv/shaders/libraries/cooperative_library.h:20-33). */
int rdv_mlp_forward(const rdv_mlp_desc* desc, const void* packed, const float* x,
                    float* y, int64_t n, void* stream);

/* Bytes of workspace rdv_mlp_forward_unpacked needs for `desc`: 0 when a
 * compile-time kernel serves the chain and every hidden width is a multiple of
 * 32 (the kernel then builds its LDS fragments from the parameters itself),
 * else rdv_mlp_packed_bytes(desc) (< 0 on error). */
int64_t rdv_mlp_unpacked_workspace_bytes(const rdv_mlp_desc* desc);

/* rdv_mlp_forward from the layers' own parameters -- weights[i] fp32 row-major
 * [dims[i+1], dims[i]], biases[i] fp32 [dims[i+1]], device pointers in host
 * arrays, as rdv_mlp_pack takes them -- read at every call, so any update of a
 * parameter buffer is seen by the next call.  Chains with a compile-time
 * kernel: one launch (each block converts W into its LDS fragments), plus the
 * exact-fp32 launch of a partial last 32-row group, which reads W directly;
 * no workspace.  Other chains: packed into `workspace` (256-byte aligned,
 * rdv_mlp_unpacked_workspace_bytes bytes; RDV_ERR_WORKSPACE when smaller) by
 * one pack launch, then rdv_mlp_forward.  Same results as rdv_mlp_pack +
 * rdv_mlp_forward.  Replaces Map.__call__ -> dispatch(MapEvaluator), whose
 * LinearFast reads the weights through their buffer pointers at every dispatch
 * (src/rdv/maths/__init__.py:1451-1487, src/rdv/shaders/maps/linear_fast.h:39-60). */
int rdv_mlp_forward_unpacked(const rdv_mlp_desc* desc, const float* const* weights, const float* const* biases,
                             const float* x, float* y, int64_t n, void* workspace, int64_t workspace_bytes,
                             void* stream);

/* Same as rdv_mlp_forward but evaluates every row (tail included) on the fp16
 * matrix-core path; exposed for benchmarking the kernel alone. */
int rdv_mlp_forward_f16_all(const rdv_mlp_desc* desc, const void* packed,
                            const float* x, float* y, int64_t n, void* stream);

/* Name of the kernel rdv_mlp_forward would launch for `desc` (for profiling
 * reports); "" if the descriptor is invalid. */
const char* rdv_mlp_kernel_name(const rdv_mlp_desc* desc);

/* ------------------------------------------------- Winograd F(2x2,3x3) conv */
/* Image layouts (one image = batch element): HWC is the reference's
 * channels-last [H*W, C] (src/rdv/domain/nn.py:1018-1024); CHW is NCHW. */
enum { RDV_LAYOUT_HWC = 0, RDV_LAYOUT_CHW = 1 };
enum { RDV_DTYPE_F32 = 0, RDV_DTYPE_F16 = 1 };
/* Filter layouts: RSCK is the reference's [3][3][CIN][COUT]; KCRS is PyTorch OIHW. */
enum { RDV_WLAYOUT_RSCK = 0, RDV_WLAYOUT_KCRS = 1 };

typedef struct rdv_conv_desc {
  int32_t batch;               /* images, stored back to back          */
  int32_t H, W;                /* even                                  */
  int32_t cin;                 /* 1..64                                 */
  int32_t cout;                /* multiple of 16, <= 1024               */
  int32_t in_layout, in_dtype; /* RDV_LAYOUT_*, RDV_DTYPE_*             */
  int32_t out_layout, out_dtype;
  int32_t relu;                /* 1: max(y, 0) after the bias           */
} rdv_conv_desc;

/* Host-only shape check; launches nothing. */
int rdv_winograd3x3_validate(const rdv_conv_desc* desc);

/* Bytes of the transformed filter bank for (cin, cout). */
int64_t rdv_winograd3x3_weight_bytes(int32_t cin, int32_t cout);

/* U = G g G^T per (cin, cout) filter in fp32, rounded to fp16, packed for the
 * matrix cores (rdv_winograd3x3_weight_bytes bytes, 16-byte aligned).  w is a
 * device pointer to the 3x3 filters in w_layout / w_dtype.
 * Replaces _winograd_transform_weight (src/rdv/domain/nn.py:525-538). */
int rdv_winograd3x3_transform_weight(const void* w, int32_t w_layout, int32_t w_dtype, int32_t cin,
                                     int32_t cout, void* U, void* stream);

/* 'same'-padded stride-1 3x3 convolution y = conv(x, w) + bias (optionally
 * ReLU), via F(2x2,3x3) with fp16 operands and fp32 accumulation.  bias is an
 * fp32 device pointer [cout] or NULL (zero).
 * Replaces Conv2DTensorOpWinograd3x3's dispatch (src/rdv/domain/nn.py:1002-1087,
 * src/rdv/shaders/tensors/conv2d_tensor_op_winograd3x3.h:95-178).  Unlike the
 * reference (CIN, COUT <= 48, (H/2)(W/2) % 32 == 0, nn.py:1066-1078) any even
 * H, W and CIN <= 64 are accepted. */
int rdv_winograd3x3_forward(const rdv_conv_desc* desc, const void* x, const void* U, const float* bias,
                            void* y, void* stream);

/* ------------------------------------------------------ tensor operations */
/* Storage of a linear tensor op's weight:
 *   F32        fp32 [out][in] (PyTorch nn.Linear layout), read at every dispatch;
 *   F16        fp16 [out][in] (LinearTensorOpSimple's pre-cast copy, nn.py:493-501);
 *   F16_TILED16 fp16 [out/16][in/16][16 k][16 n] (LinearTensorOpFast's pre-tiled
 *              copy, nn.py:472-490). */
enum { RDV_WKIND_F32 = 0, RDV_WKIND_F16 = 1, RDV_WKIND_F16_TILED16 = 2 };

typedef struct rdv_linear_op_desc {
  int64_t rows;          /* batch rows of x and y (>= 0)                            */
  int32_t in_features;   /* multiple of 8                                           */
  int32_t out_features;  /* multiple of 4                                           */
  int32_t precision;     /* RDV_PREC_F16: x and W rounded to fp16, fp32 accumulation
                            (LinearTensorOp{Small,Simple,Fast,Mine}); RDV_PREC_F32:
                            fp32 throughout (LinearTensorOp)                        */
  int32_t wkind;         /* RDV_WKIND_*; F16 kinds need RDV_PREC_F16                */
  int32_t relu;          /* 1: y = max(y, 0) after the bias (build-defined fusion; the
                            reference's tensor-op path has a separate ReLUTensorOp)  */
  int32_t reserved;      /* 0                                                       */
} rdv_linear_op_desc;

/* Host-only shape check; launches nothing. */
int rdv_linear_op_validate(const rdv_linear_op_desc* desc);

/* y[rows, out] = x[rows, in] W^T + bias, fp32 x / bias / y (16-byte aligned device
 * pointers), weight per desc->wkind (16-byte aligned for F32 and F16).
 * Replaces the dispatch of LinearTensorOp (src/rdv/domain/nn.py:377-411,
 * src/rdv/shaders/tensors/linear_tensor_op.h:8-51), LinearTensorOpSmall
 * (nn.py:1303-1411, linear_tensor_op_small.h:50-247), LinearTensorOpSimple
 * (nn.py:1204-1300, linear_tensor_op_simple.h:49-116), LinearTensorOpFast
 * (nn.py:541-605, linear_tensor_op_fast.h:37-122) and LinearTensorOpMine
 * (nn.py:1153-1201, linear_tensor_op_mine.h:51-133), all through
 * TensorOpEvaluator (src/rdv/maths/__init__.py:1382-1399). */
int rdv_linear_op(const rdv_linear_op_desc* desc, const float* x, const void* weight, const float* bias, float* y,
                  void* stream);

/* y[i] = max(x[i], 0) for i < n (fp32, 16-byte aligned; a NaN maps to 0).
 * Replaces ReLUTensorOp (src/rdv/domain/nn.py:362-374,
 * src/rdv/shaders/tensors/relu_tensor_op.h:3-22). */
int rdv_relu_op(const float* x, float* y, int64_t n, void* stream);

/* Direct 2-D convolution of a KH x KW kernel, stride 1, 'same' zero padding
 * (KH / 2 rows above, KW / 2 columns to the left, the rest below / right),
 * over a channels-last fp32 image x[H*W, cin] -> y[H*W, cout] fp32. */
typedef struct rdv_conv2d_desc {
  int32_t H, W;       /* image size (>= 0)                                         */
  int32_t cin;        /* >= 1 (multiples of 8 for fp16, 4 for fp32, take 16-byte
                         gathers; others a per-element gather)                     */
  int32_t cout;       /* >= 1 (multiples of 4 take 16-byte stores)                  */
  int32_t kh, kw;     /* kernel size, 1..31                                         */
  int32_t precision;  /* RDV_PREC_F16: x and w rounded to fp16, fp32 accumulation;
                         RDV_PREC_F32: fp32 throughout                              */
  int32_t w_layout;   /* RDV_WLAYOUT_RSCK [kh][kw][cin][cout] (the tensor ops') or
                         RDV_WLAYOUT_KCRS [cout][cin][kh][kw] (PyTorch, Conv2dGrid) */
  int32_t relu;       /* 1: y = max(y, 0) after the bias (build-defined fusion)     */
  int32_t reserved;   /* 0                                                          */
} rdv_conv2d_desc;

/* Host-only shape check; launches nothing. */
int rdv_conv2d_validate(const rdv_conv2d_desc* desc);

/* y = conv(x, w) + bias: y[p][o] = bias[o] + sum over taps (kh, kw) inside the
 * image and channels c of x[tap pixel][c] * w[kh][kw][c][o], the taps in (kh,
 * kw) order and channels ascending (fp32 association order otherwise
 * unspecified).  x, y: fp32 device pointers (16-byte aligned for the vector
 * path, 4-byte otherwise); w: fp32 device
 * pointer in desc->w_layout, read at every call; bias: fp32 [cout] or NULL.
 * Replaces the dispatches of Conv2DTensorOp (src/rdv/domain/nn.py:414-470,
 * src/rdv/shaders/tensors/conv2d_tensor_op.h:20-80; RDV_PREC_F32) and of
 * Conv2DTensorOpFast, Conv2DTensorOpSimple, Conv2DTensorOpSimple3x3 and
 * Conv2DTensorOpWindow3x3 (nn.py:608-1000, shaders/tensors/conv2d_tensor_op_
 * {fast,simple,simple3x3,window3x3}.h; RDV_PREC_F16), and of the grid
 * convolutions Conv2dGrid / Conv2D (nn.py:122-266, shaders/grids/conv2d.h,
 * conv2d_per_output.h) over a materialised input grid. */
int rdv_conv2d(const rdv_conv2d_desc* desc, const float* x, const float* w, const float* bias, float* y,
               void* stream);

/* Data movement over channels-last fp32 images x[H*W, C] (any C >= 1; C a
 * multiple of 4 with 16-byte aligned x and y takes 16-byte accesses; the
 * reference's tensor ops ask C % 8 == 0 and row counts that are multiples of
 * 4, which the Python classes keep; its grid versions take any C).
 * y[(H/2)*(W/2), C] = 2x2 average pool, stride 2: ((x00 + x01) + x10) + x11
 * summed left to right in fp32, times 0.25 (H, W even).
 * Replaces Downsample2xTensorOp (src/rdv/domain/nn.py:1090-1107,
 * src/rdv/shaders/tensors/downsample2x_tensor_op.h:1-37). */
int rdv_downsample2x(const float* x, int64_t H, int64_t W, int32_t C, float* y, void* stream);

/* y[(2H)*(2W), C]: nearest-neighbour 2x upsample of x[H*W, C].
 * Replaces Upsample2xTensorOp (src/rdv/domain/nn.py:1110-1125,
 * src/rdv/shaders/tensors/upsample2x_tensor_op.h:1-29). */
int rdv_upsample2x(const float* x, int64_t H, int64_t W, int32_t C, float* y, void* stream);

/* y[rows, C1 + C2] = [x1[rows, C1] | x2[rows, C2]] (C1, C2 multiples of 4).
 * Replaces ConcatTensorOp (src/rdv/domain/nn.py:1128-1150,
 * src/rdv/shaders/tensors/concat_tensor_op.h:1-25). */
int rdv_concat_channels(const float* x1, int32_t C1, const float* x2, int32_t C2, int64_t rows, float* y,
                        void* stream);

/* ------------------------------------------------- MLP training step (C5) */
/* Bytes of workspace rdv_mlp_train_step needs for `desc` and n points (< 0 if
 * the chain is not supported by the training kernels). */
int64_t rdv_mlp_train_workspace_bytes(const rdv_mlp_desc* desc, int64_t n);

/* Forward + MSE loss + backward of a LinearFast / ReLU chain (build-defined;
 * the reference has no backward pass).  x: device [n, dims[0]] fp16; target:
 * device [n, dims[L]] fp32; loss: device fp32 scalar = mean over n x dims[L] of
 * (y - target)^2; dW[i] / db[i] (host arrays of device pointers): fp32
 * [dims[i+1], dims[i]] / [dims[i+1]] gradients of the loss, reduced over every
 * point in fp32.  Supported chains: ReLU hidden layers, linear head, input
 * width a multiple of 16 and hidden widths multiples of 32 (all <= 128), head
 * width a multiple of 8 (<= 128).  workspace: rdv_mlp_train_workspace_bytes
 * bytes, 256-byte aligned. */
int rdv_mlp_train_step(const rdv_mlp_desc* desc, const void* packed, const void* x, const float* target, int64_t n,
                       void* workspace, int64_t workspace_bytes, float* loss, float* const* dW, float* const* db,
                       void* stream);

/* Size of the static device scratch behind rdv_mlp_train_step_static. */
#define RDV_TRAIN_STATIC_SCRATCH_BYTES (64LL << 20)

/* rdv_mlp_train_step without a workspace argument and without any device
 * allocation: the workspace is a file-scope device array of
 * RDV_TRAIN_STATIC_SCRATCH_BYTES bytes, one per GPU, held until the process
 * ends.  No counterpart in the reference (which has no backward pass); it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as rdv_mlp_train_step.  Returns
 * RDV_ERR_WORKSPACE when rdv_mlp_train_workspace_bytes(desc, n) exceeds the
 * scratch size.  Every call on one GPU shares that GPU's scratch: calls that
 * overlap on one GPU (two streams, two threads) race. */
int rdv_mlp_train_step_static(const rdv_mlp_desc* desc, const void* packed, const void* x, const float* target,
                              int64_t n, float* loss, float* const* dW, float* const* db, void* stream);

/* ------------------------------------------------ cameras and volume rendering */
typedef struct rdv_camera_desc {
  int32_t n_cams;       /* poses rows                                             */
  int32_t width, height;
  float aspect_ratio;   /* reference default width / height                       */
  float fov;            /* vertical field of view in radians (reference default pi/4) */
} rdv_camera_desc;

/* rays[n, H, W, 6] = (origin, unit direction) of the pinhole camera ray through
 * each pixel centre; poses is a device [n, 9] fp32 array (origin | target | up).
 * Replaces Cameras' grid dispatch (src/rdv/domain/rendering.py:10-42,
 * src/rdv/shaders/rendering/cameras.h:1-20) with pixel_jitter == 0. */
int rdv_cameras_rays(const rdv_camera_desc* cam, const float* poses, float* rays, void* stream);

/* rdv_cameras_rays with pixel jitter (Cameras(jitter=True), cameras.h:7): the
 * ray of cell i (the row-major cell index) passes through sub-pixel position
 * (u0, u1) instead of the centre, where u0, u1 are the first two random()
 * values of thread i of a dispatch with these seeds (rdv_random_uniform).
 * seeds: 4 host words (RandomLibrary's per-dispatch uvec4). */
int rdv_cameras_rays_jittered(const rdv_camera_desc* cam, const float* poses, const uint32_t* seeds, float* rays,
                              void* stream);

/* ----------------------------------------------------- batched grid evaluation */
#define RDV_GRID_MAX_RANK 8

/* rays[i] = the camera ray of the index vector indices[i] = (cam, y, x), for a
 * device int32 [n, 3] batch: the batch branch of Grid.__call__ on a Cameras
 * grid (src/rdv/maths/__init__.py:104-119,
 * src/rdv/shaders/grids/batch_grid_evaluator.h, rendering/cameras.h:1-20).
 * seeds == NULL: pixel centres; else 4 host words, and row i draws its
 * sub-pixel position from thread i's generator (the batch row is the
 * reference batch evaluator's thread index).  cam outside [0, n_cams) gives a
 * row of NaN; y and x are used as given.  n may be 0. */
int rdv_cameras_rays_at(const rdv_camera_desc* cam, const float* poses, const int32_t* indices, int64_t n,
                        const uint32_t* seeds, float* rays, void* stream);

/* out[i, :] = values[cell(indices[i]), :] for a grid of `rank` dimensions
 * (shape: host array) whose cells hold `width` fp32 values, row-major with the
 * last dimension fastest (grid_library.h:3-16), and a device int32 [n, rank]
 * batch of index vectors: the batch branch of Grid.__call__ over materialised
 * grid values (TensorGrid's forward, src/rdv/shaders/grids/tensor_grid.h,
 * behind BatchGridEvaluator, src/rdv/maths/__init__.py:815-844).  An index
 * outside its dimension gives a row of NaN.  n may be 0. */
int rdv_grid_gather(const float* values, int32_t rank, const int64_t* shape, int32_t width, const int32_t* indices,
                    int64_t n, float* out, void* stream);

/* out[t * per_thread + k] = the k-th random() value of thread t of a dispatch
 * whose seeds are `seeds` (4 host words): the reference's per-thread generator
 * (three Tausworthe steps and an LCG, GPU Gems 3 ch. 37), spawned from the
 * seeds and thread index t and mapped to [0, 1) through the mantissa
 * (src/rdv/shaders/libraries/random_library.h:1-62, :255-267;
 * src/rdv/core/_common.py:56-89).  n_threads < 2^31. */
int rdv_random_uniform(const uint32_t* seeds, int64_t n_threads, int32_t per_thread, float* out, void* stream);

/* Emission-absorption render of a density / RGB field (build-defined; no
 * reference counterpart): for every pixel ray of `cam` that meets [-1,1]^3 on
 * [t0, t1] (t0 >= 0), `samples` points t_i = t0 + (i + 1/2) dt, dt = (t1 - t0) /
 * samples, are evaluated by `field` (a LinearFast chain from 3 inputs to 4 raw
 * outputs; sigma = softplus(o0), c = sigmoid(o1..3)) and composited
 * front to back: alpha_i = 1 - exp(-sigma_i dt), T_i = prod_{j<i} (1 - alpha_j),
 * image = sum_i T_i alpha_i c_i (0 for rays that miss).  image: device
 * [n, H, W, 3] fp32.  samples: a positive multiple of 32. */
int rdv_render_emission_absorption(const rdv_camera_desc* cam, const float* poses, const rdv_mlp_desc* field,
                                   const void* packed, int32_t samples, float* image, void* stream);

/* rdv_render_emission_absorption over rays given in memory: rays[n_rays, 6] =
 * (origin, direction) fp32, out[n_rays, 3] (EmissionAbsorption as a Map[6, 3]
 * over any grid of rays; build-defined). */
int rdv_render_emission_absorption_rays(const rdv_mlp_desc* field, const void* packed, const float* rays,
                                        int64_t n_rays, int32_t samples, float* out, void* stream);

/* The same compositing over precomputed samples (build-defined):
 * sigma_rgb[n_rays, samples, 4] = (sigma, r, g, b), dt[n_rays] the sample
 * spacing of each ray (0 for rays that miss), out[n_rays, 3]. */
int rdv_composite(const float* sigma_rgb, const float* dt, int64_t n_rays, int32_t samples, float* out,
                  void* stream);

/* out[n] = transmittance along each ray rays[n, 6] = (x, w) through the box
 * [-1,1]^3 in the object space of transform (mat4x3, column-major: three linear
 * columns then the translation, 12 floats on the host), marched with fixed
 * steps of step_size: tau += extinction(x) * density_scale * step_size, 0 once
 * tau > 16, exp(-tau) at the end (1 for rays that miss).  extinction: any
 * LinearFast chain from 3 inputs to 1 output (the reference marches any
 * extinction Map[3, 1]).
 * Replaces RaymarchingTransmittance (src/rdv/domain/volumes.py:124-141,
 * src/rdv/shaders/volumes/raymarching_transmittance.h:1-22,
 * raymarching_transmittance_trait.h:1-14, libraries/math_library.h:48-57). */
int rdv_raymarch_transmittance(const rdv_mlp_desc* extinction, const void* packed, const float* rays,
                               int64_t n_rays, const float* transform12, float step_size, float density_scale,
                               float* out, void* stream);

/* ------------------------------------------------ ratio tracking and majorants */
typedef struct rdv_ratiotracking_desc {
  float transform[12];   /* mat4x3, column-major, as rdv_raymarch_transmittance      */
  float density_scale;
  int32_t maj_width, maj_height, maj_depth;  /* the majorant grid [depth, height, width] */
  uint32_t seeds[4];     /* the dispatch's random seeds                              */
  int32_t rng_skip;      /* random() draws each thread took before this map (2 when the
                            rays come from a jittered camera of the same dispatch)   */
  int32_t reserved;      /* 0                                                        */
} rdv_ratiotracking_desc;

/* out[n] = ratio-tracking transmittance along each ray rays[n, 6] = (x, w)
 * through the box [-1,1]^3 in the object space of the transform, with a voxel
 * majorant field: free flights of -log(1 - random()) / (majorant * density_scale)
 * capped at the voxel exit, T *= 1 - extinction(x) / majorant at each
 * collision, Russian roulette below T = 0.05, at most 1024 steps (1 for rays
 * that miss).  Thread i (ray i) draws from the generator of rdv_random_uniform
 * with rt->seeds, after skipping rt->rng_skip values.  majorant: device
 * [depth, height, width] fp32, every value an upper bound of the extinction over
 * its voxel (else the estimate is biased).  extinction: any LinearFast chain from
 * 3 inputs to 1 output.
 * Replaces RatiotrackingTransmittance with VoxelMajorantField
 * (src/rdv/domain/volumes.py:144-211, shaders/volumes/ratiotracking_transmittance.h,
 * ratiotracking_transmittance_trait.h:1-31, voxel_majorant_field.h:1-33). */
int rdv_ratiotracking_transmittance(const rdv_mlp_desc* extinction, const void* packed,
                                    const rdv_ratiotracking_desc* rt, const float* majorant, const float* rays,
                                    int64_t n_rays, float* out, void* stream);

/* VoxelMajorantField as a Map[6, 2] over rows: out[i] = (the value of the grid
 * voxel holding x_i, the distance along w_i to that voxel's exit), rays[n, 6] in
 * the grid's [-1,1]^3 box; grid: device [depth, height, width] fp32
 * (src/rdv/domain/volumes.py:191-211, shaders/volumes/voxel_majorant_field.h:1-33). */
int rdv_voxel_majorant(const float* grid, int32_t width, int32_t height, int32_t depth, const float* rays,
                       int64_t n_rays, float* out, void* stream);

typedef struct rdv_majorant_grid_desc {
  int32_t rank;           /* grid dimensions, 1..4                                  */
  int32_t channels;       /* values per cell (the grid's OUT)                       */
  int32_t fine_shape[4];  /* the wrapped grid's shape (first `rank` entries)        */
  int32_t shape[4];       /* the majorant grid's shape                              */
  int32_t aligned;        /* the sampler convention: 1 ties -1/+1 to the outer voxel centres */
  int32_t linear;         /* 1: interpolating sampler (reaches one more voxel)      */
} rdv_majorant_grid_desc;

/* out[shape..., channels] = per coarse cell, the channel-wise maximum over every
 * fine cell that a sampler with the given aligned / linear convention could read
 * from inside that coarse cell; fine: device [fine_shape..., channels] fp32.
 * Replaces MajorantGrid (src/rdv/maths/__init__.py:534-569,
 * shaders/grids/majorant_grid.h). */
int rdv_majorant_grid(const rdv_majorant_grid_desc* desc, const float* fine, float* out, void* stream);

/* ------------------------------------------------------------- volume profile */
#define RDV_VP_MAX_DEPTH 16    /* transmittance thresholds (DEPTH_SAMPLES)   */
#define RDV_VP_MAX_SPECTRAL 8  /* SPECTRAL_DIM                               */

typedef struct rdv_volume_profile_desc {
  float transform[12];         /* mat4x3, column-major, as rdv_raymarch_transmittance     */
  float density_scale;
  float g;                     /* Henyey-Greenstein anisotropy                           */
  float step_size;             /* fixed step of the marches                              */
  float light_direction[3];    /* world space                                            */
  float light_intensity[RDV_VP_MAX_SPECTRAL];
  float transmittance_threshold[RDV_VP_MAX_DEPTH];
  int32_t depth_samples;       /* DEPTH_SAMPLES, 1..RDV_VP_MAX_DEPTH                     */
  int32_t spectral_dim;        /* SPECTRAL_DIM, 1..RDV_VP_MAX_SPECTRAL                   */
  int32_t sample_index;        /* the depth sample whose position is shaded, 0..depth_samples-1 */
  int32_t environment_samples; /* >= 0                                                   */
  int32_t maj_width, maj_height, maj_depth;  /* the voxel majorant grid [depth, height, width] */
  uint32_t seeds[4];           /* the dispatch's random seeds                            */
  int32_t rng_skip;            /* random() draws each thread took before this map        */
  int32_t reserved;            /* 0                                                      */
} rdv_volume_profile_desc;

/* VolumeProfile, first stage: per ray rays[n, 6] = (x, w), everything but the
 * two spectral maps.  In the object space of the transform: the ray's box
 * [-1,1]^3 interval trimmed at both ends while the voxel majorant is 0; tau by
 * a fixed-step march (left endpoints, stop past 20); a second march that
 * records the depth t where tau crosses each threshold's expected crossing
 * value; S = 1 - exp(-tau); the depths re-encoded; then at the sample depth's
 * position the light ray's raymarched transmittance and, per environment
 * sample, a Henyey-Greenstein direction and its ratio-tracked transmittance
 * (thread i = ray i draws from rdv_random_uniform's generator with vp->seeds
 * after vp->rng_skip draws).  out[n, 4 + 3 SD + DS] receives every output
 * except the environment and albedo features; per ray, sample_pos[n, 3] gets
 * the object-space sample position, env_dirs[n, ES, 3] each environment
 * direction (world space), env_weights[n, ES] = S * T of each, valid[n] 1 where
 * the ray reached at least one depth (0 elsewhere: those rows are final).
 * extinction: any LinearFast chain from 3 inputs to 1 output; majorant: device
 * [depth, height, width] fp32 of a VoxelMajorantField.
 * Replaces VolumeProfile's shader (src/rdv/domain/volumes.py:503-550,
 * shaders/volumes/volume_profile.h:1-167 and the traits it calls:
 * raymarching_transmittance_trait.h, ratiotracking_transmittance_trait.h,
 * voxel_majorant_field.h, random_library.h:224-239 hg_phase_sample,
 * math_library.h:48-57, 323-330). */
int rdv_volume_profile(const rdv_mlp_desc* extinction, const void* packed, const rdv_volume_profile_desc* vp,
                       const float* majorant, const float* rays, int64_t n_rays, float* out, float* sample_pos,
                       float* env_dirs, float* env_weights, int32_t* valid, void* stream);

/* VolumeProfileDDA, first stage: as rdv_volume_profile, except the tau and
 * depth marches.  Those do not trim the ray's ends.  Instead they walk
 * majorant_grid (device [grid_depth, grid_height, grid_width] fp32 over the
 * box, e.g. rdv_majorant_grid's output) cell by cell with an Amanatides-Woo
 * DDA from the entry cell: at most 4096 cells, until tMax or off the grid.
 * In a cell whose value is > 0 the march samples t, t + step, ... while t is
 * below the cell's exit, then t jumps to the exit; cells whose value is not
 * > 0 are skipped whole.  `majorant` (the VoxelMajorantField's grid) still
 * serves the environment rays' ratio tracking.  Grid dimensions 1..4096.
 * Replaces VolumeProfileDDA's shader (src/rdv/domain/volumes.py:560-603,
 * shaders/volumes/volume_profile_dda.h:1-208). */
int rdv_volume_profile_dda(const rdv_mlp_desc* extinction, const void* packed, const rdv_volume_profile_desc* vp,
                           const float* majorant, const float* majorant_grid, int32_t grid_width,
                           int32_t grid_height, int32_t grid_depth, const float* rays, int64_t n_rays, float* out,
                           float* sample_pos, float* env_dirs, float* env_weights, int32_t* valid, void* stream);

/* VolumeProfile, second stage, for rows with valid[i] = 1: the environment
 * feature out[i, DS+2+c] = sum over s of env_weights[i, s] * env[i ES + s, c] / ES
 * (accumulated in s order) and the albedo feature out[i, DS+2+SD+c] =
 * 1 / (1 - log(1 - albedo[i, c])), where env and albedo are the
 * ENVIRONMENT and SCATTERING_ALBEDO maps evaluated at env_dirs and sample_pos
 * (row strides env_stride / albedo_stride floats; 0 repeats one row, for a
 * constant map).  Replaces volume_profile.h:155-160. */
int rdv_volume_profile_finish(const rdv_volume_profile_desc* vp, const float* albedo, int64_t albedo_stride,
                              const float* env, int64_t env_stride, const float* env_weights,
                              const int32_t* valid, int64_t n_rays, float* out, void* stream);

/* out[rows, width] = value[width] repeated on every row: a Constant map over
 * rows (src/rdv/maths/__init__.py:1659-1668, shaders/maps/constant.h). */
int rdv_broadcast_rows(const float* value, int32_t width, int64_t rows, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* RDV_HIP_H */
