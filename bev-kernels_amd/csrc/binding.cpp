// C ABI of libbevk.so: argument validation, error reporting and dispatch onto the
// kernel launchers. The entry points keep the argument order of the reference's
// pybind11 functions (naotic/bev-kernels csrc/binding.cpp:142-191 and
// csrc_musa/msda/binding_musa.mu:545-557) with tensors lowered to device pointers.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/bev_kernels.h"
#include "bevk_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() { return BEVK_OK; }

int hip_status(hipError_t e, const char *what) {
  if (e == hipSuccess) return ok();
  return fail(BEVK_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

const char *dtype_name(int dtype) {
  switch (dtype) {
    case BEVK_F32: return "Float";
    case BEVK_F16: return "Half";
    case BEVK_BF16: return "BFloat16";
    case BEVK_F64: return "Double";
    default: return "unknown";
  }
}

bool valid_dtype(int dtype) { return dtype >= BEVK_F32 && dtype <= BEVK_F64; }

int dtype_size(int dtype) {
  switch (dtype) {
    case BEVK_F32: return 4;
    case BEVK_F16: case BEVK_BF16: return 2;
    default: return 8;
  }
}

// The kernels address one image (or, for the fused kernel, the whole input) through a
// 32-bit buffer range with an out-of-range sentinel just past its end.
constexpr long long kMaxBufferBytes = (1LL << 31) - 256;

// Shared geometry checks of the DCN entry points; the output size must follow the
// convolution formula (modulated_deform_conv.py:364-365).
int check_geom(const char *fn, const bevk::DcnGeom &g) {
  if (g.batch < 0 || g.channels < 0 || g.height < 0 || g.width < 0)
    return fail(BEVK_ERR_INVALID, "%s: negative input size", fn);
  if (g.kernel_h <= 0 || g.kernel_w <= 0 || g.stride_h <= 0 || g.stride_w <= 0 ||
      g.dil_h <= 0 || g.dil_w <= 0 || g.pad_h < 0 || g.pad_w < 0)
    return fail(BEVK_ERR_INVALID,
                "%s: kernel, stride and dilation must be positive and padding non-negative", fn);
  if (g.deformable_group <= 0)
    return fail(BEVK_ERR_INVALID, "%s: deformable_group must be positive", fn);
  if (g.channels % g.deformable_group != 0)
    return fail(BEVK_ERR_INVALID, "%s: channels (%d) must be divisible by deformable_group (%d)",
                fn, g.channels, g.deformable_group);
  const int ho = (g.height + 2 * g.pad_h - (g.dil_h * (g.kernel_h - 1) + 1)) / g.stride_h + 1;
  const int wo = (g.width + 2 * g.pad_w - (g.dil_w * (g.kernel_w - 1) + 1)) / g.stride_w + 1;
  if (g.height_col != ho || g.width_col != wo)
    return fail(BEVK_ERR_INVALID,
                "%s: output size (%d, %d) does not match the convolution geometry (%d, %d)", fn,
                g.height_col, g.width_col, ho, wo);
  if (ho <= 0 || wo <= 0)
    return fail(BEVK_ERR_INVALID, "%s: empty output (%d x %d)", fn, ho, wo);
  return ok();
}

bevk::DcnGeom make_geom(int batch_size, int channels, int height_im, int width_im,
                        int height_col, int width_col, int kernel_h, int kernel_w, int pad_h,
                        int pad_w, int stride_h, int stride_w, int dilation_h, int dilation_w,
                        int deformable_group) {
  bevk::DcnGeom g;
  g.batch = batch_size; g.channels = channels; g.height = height_im; g.width = width_im;
  g.height_col = height_col; g.width_col = width_col;
  g.kernel_h = kernel_h; g.kernel_w = kernel_w; g.pad_h = pad_h; g.pad_w = pad_w;
  g.stride_h = stride_h; g.stride_w = stride_w; g.dil_h = dilation_h; g.dil_w = dilation_w;
  g.deformable_group = deformable_group;
  return g;
}

int im2col_nchw_common(const char *fn, bool tiled, int dtype, const void *data_im,
                       const void *data_offset, const void *data_mask, const bevk::DcnGeom &g,
                       void *data_col, void *stream) {
  g_last_error.clear();
  if (!valid_dtype(dtype)) return fail(BEVK_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (int rc = check_geom(fn, g)) return rc;
  const long long cols = (long long)g.channels * g.kernel_h * g.kernel_w * g.batch *
                         g.height_col * g.width_col;
  if (cols == 0) return ok();
  if ((long long)g.channels * g.height * g.width * dtype_size(dtype) > kMaxBufferBytes)
    return fail(BEVK_ERR_INVALID, "%s: one input image exceeds 2 GiB", fn);
  if (!data_im || !data_offset || !data_mask || !data_col)
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_im2col_nchw(dtype, g, data_im, data_offset, data_mask,
                                             data_col, tiled, (hipStream_t)stream),
                    fn);
}

}  // namespace

extern "C" {

const char *bevk_last_error(void) { return g_last_error.c_str(); }

const char *bevk_version(void) { return "bevk 0.1.0 gfx950"; }

int bevk_modulated_deformable_im2col(int dtype, const void *data_im, const void *data_offset,
                                     const void *data_mask, int batch_size, int channels,
                                     int height_im, int width_im, int height_col, int width_col,
                                     int kernel_h, int kernel_w, int pad_h, int pad_w,
                                     int stride_h, int stride_w, int dilation_h, int dilation_w,
                                     int deformable_group, void *data_col, void *stream) {
  return im2col_nchw_common(
      "modulated_deformable_im2col", false, dtype, data_im, data_offset, data_mask,
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                deformable_group),
      data_col, stream);
}

int bevk_modulated_deformable_im2col_opt(
    int dtype, const void *data_im, const void *data_offset, const void *data_mask,
    int batch_size, int channels, int height_im, int width_im, int height_col, int width_col,
    int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
    int dilation_h, int dilation_w, int deformable_group, void *data_col, void *stream) {
  return im2col_nchw_common(
      "modulated_deformable_im2col_opt", true, dtype, data_im, data_offset, data_mask,
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                deformable_group),
      data_col, stream);
}

int bevk_modulated_deformable_im2col_nhwc(
    int dtype, const void *data_im, const void *data_offset, int offset_last_dim,
    const void *data_mask, int batch_size, int channels, int height_im, int width_im,
    int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *data_col, void *stream) {
  const char *fn = "modulated_deformable_im2col_nhwc";
  g_last_error.clear();
  // dcn_fused_nhwc_cuda.cu:34-35
  if (deformable_group != 1)
    return fail(BEVK_ERR_INVALID, "NHWC fused path supports deformable_group == 1 only");
  if (!valid_dtype(dtype)) return fail(BEVK_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_geom(fn, g)) return rc;
  const int taps = kernel_h * kernel_w;
  if (offset_last_dim != 2 * taps && offset_last_dim != 3 * taps)
    return fail(BEVK_ERR_INVALID, "%s: offset last dim must be 2T (%d) or 3T (%d), got %d", fn,
                2 * taps, 3 * taps, offset_last_dim);
  const bool fused_y = offset_last_dim == 3 * taps;  // dcn_fused_nhwc_cuda.cu:54
  const long long m = (long long)batch_size * height_col * width_col;
  // dcn_fused_nhwc_cuda.cu:37-40
  if (m * taps * channels >= 2147483647LL)
    return fail(BEVK_ERR_INVALID, "NHWC gather: Col element count exceeds int32 range");
  if (m * taps * channels == 0) return ok();
  if ((long long)height_im * width_im * channels * dtype_size(dtype) > kMaxBufferBytes)
    return fail(BEVK_ERR_INVALID, "%s: one input image exceeds 2 GiB", fn);
  if (!data_im || !data_offset || (!fused_y && !data_mask) || !data_col)
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_im2col_nhwc(dtype, g, data_im, data_offset, fused_y, data_mask,
                                             data_col, (hipStream_t)stream),
                    fn);
}

int bevk_modulated_deformable_col2im_nchw(
    int dtype, const void *data_col, const void *data_im, const void *data_offset,
    const void *data_mask, int batch_size, int channels, int height_im, int width_im,
    int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *grad_im, void *grad_offset, void *grad_mask, void *stream) {
  const char *fn = "modulated_deformable_col2im";
  g_last_error.clear();
  if (!valid_dtype(dtype)) return fail(BEVK_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w,
                deformable_group);
  if (int rc = check_geom(fn, g)) return rc;
  const long long n = (long long)batch_size * deformable_group * kernel_h * kernel_w *
                      height_col * width_col;
  if (n == 0 || channels == 0) return ok();
  if ((grad_offset == nullptr) != (grad_mask == nullptr))
    return fail(BEVK_ERR_INVALID, "%s: grad_offset and grad_mask go together", fn);
  if (!data_col || !data_offset || !data_mask || (!grad_im && !grad_offset) ||
      (grad_offset && !data_im))
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  // 16-bit grad_im takes packed pair atomics: its first element must start a pair
  if (grad_im && dtype_size(dtype) == 2 && reinterpret_cast<uintptr_t>(grad_im) % 4 != 0)
    return fail(BEVK_ERR_INVALID, "%s: 16-bit grad_im must be 4-byte aligned", fn);
  return hip_status(bevk::launch_col2im_nchw(dtype, g, data_col, data_im, data_offset, data_mask,
                                             grad_im, grad_offset, grad_mask,
                                             (hipStream_t)stream),
                    fn);
}

int bevk_modulated_deformable_col2im_nhwc(
    int dtype, const void *dcol, const void *data_im, const void *data_offset,
    int offset_last_dim, const void *data_mask, int batch_size, int channels, int height_im,
    int width_im, int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    float *grad_im, float *grad_offset, float *grad_mask, void *stream) {
  const char *fn = "modulated_deformable_col2im_nhwc";
  g_last_error.clear();
  if (deformable_group != 1)
    return fail(BEVK_ERR_INVALID, "NHWC fused path supports deformable_group == 1 only");
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_geom(fn, g)) return rc;
  const int taps = kernel_h * kernel_w;
  if (offset_last_dim != 2 * taps && offset_last_dim != 3 * taps)
    return fail(BEVK_ERR_INVALID, "%s: offset last dim must be 2T (%d) or 3T (%d), got %d", fn,
                2 * taps, 3 * taps, offset_last_dim);
  const bool fused_y = offset_last_dim == 3 * taps;
  const long long m = (long long)batch_size * height_col * width_col;
  if (m * taps * channels >= 2147483647LL)
    return fail(BEVK_ERR_INVALID, "NHWC col2im: Col element count exceeds int32 range");
  if (m * taps == 0) return ok();
  if ((grad_offset == nullptr) != (grad_mask == nullptr))
    return fail(BEVK_ERR_INVALID, "%s: grad_offset and grad_mask go together", fn);
  if (!dcol || !data_offset || (!fused_y && !data_mask) || (!grad_im && !grad_offset) ||
      (grad_offset && !data_im))
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_col2im_nhwc(dtype, g, dcol, data_im, data_offset, fused_y,
                                             data_mask, grad_im, grad_offset, grad_mask,
                                             (hipStream_t)stream),
                    fn);
}

// Static scratch of the allocation-free front end
// (bevk_modulated_deformable_fused_im2col_nhwc_noalloc): the packed offset-conv weight and
// the fp32 offset-conv output y [M][3T] of one call. Every GPU the library runs on holds
// its own copy until the process ends; calls that overlap on one GPU share it and race.
static constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

// The device address of `scratch` on the current device, looked up once per device (the
// host-side name is not a device address: kernels and copies take this pointer).
static constexpr int kMaxScratchDevices = 64;
static std::mutex g_scratch_mutex;
static void *g_scratch_ptr[kMaxScratchDevices];

static int device_scratch(const char *fn, void **out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices)
    return fail(BEVK_ERR_HIP, "%s: no usable current HIP device", fn);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void *ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(BEVK_ERR_HIP, "%s: hipGetSymbolAddress(scratch) failed: %s", fn,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

// Workspace of the fused front end: packed offset-conv weight, then y [M][3T] fp32.
static long long fused_im2col_ws_parts(int dtype, long long m, int taps, int channels,
                                       long long *y_offset) {
  const long long packed = bevk::dcn_packed_weight_elems(dtype, 3 * taps, taps * channels) *
                           dtype_size(dtype);
  *y_offset = (packed + 255) / 256 * 256;
  return *y_offset + m * 3 * taps * (long long)sizeof(float);
}

int64_t bevk_dcn_fused_im2col_nhwc_workspace_bytes(int dtype, int batch_size, int channels,
                                                   int height_col, int width_col, int kernel_h,
                                                   int kernel_w) {
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16) return -1;
  if (batch_size < 0 || channels < 0 || height_col < 0 || width_col < 0 || kernel_h <= 0 ||
      kernel_w <= 0)
    return -1;
  long long y_offset = 0;
  return fused_im2col_ws_parts(dtype, (long long)batch_size * height_col * width_col,
                               kernel_h * kernel_w, channels, &y_offset);
}

// The fused front end (offset conv + sigmoid + gather into the columns) with its scratch
// in the caller's `workspace`, or (static_scratch) in the library's static scratch, whose
// capacity is then workspace_bytes: a larger need is an error.
static int fused_im2col_run(
    const char *fn, bool static_scratch, int dtype, const void *data_im, const void *w_off, const float *b_off,
    int batch_size, int channels, int height_im, int width_im, int height_col, int width_col,
    int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
    int dilation_h, int dilation_w, int deformable_group, void *workspace,
    int64_t workspace_bytes, void *data_col, void *stream) {
  g_last_error.clear();
  // dcn_fused_nhwc_cuda.cu:99-100
  if (deformable_group != 1)
    return fail(BEVK_ERR_INVALID, "NHWC fused path supports deformable_group == 1 only");
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_geom(fn, g)) return rc;
  const int taps = kernel_h * kernel_w;
  if (dtype != BEVK_F32 && taps > 9)
    return fail(BEVK_ERR_UNSUPPORTED,
                "%s: kernels of more than 9 taps are fp32-only (use the split path)", fn);
  const long long m = (long long)batch_size * height_col * width_col;
  // dcn_fused_nhwc_cuda.cu:101-103
  if (m * taps * channels >= 2147483647LL)
    return fail(BEVK_ERR_INVALID, "NHWC fused: Col element count exceeds int32 range");
  if (m * taps * channels == 0) return ok();
  const int vec = 16 / dtype_size(dtype);
  if (channels % vec != 0)
    return fail(BEVK_ERR_UNSUPPORTED,
                "%s: channels (%d) must be a positive multiple of %d for '%s'", fn, channels,
                vec, dtype_name(dtype));
  if ((long long)batch_size * height_im * width_im * channels * dtype_size(dtype) >
          kMaxBufferBytes ||
      m >= (1LL << 30))
    return fail(BEVK_ERR_INVALID, "%s: problem too large for 32-bit buffer offsets", fn);
  long long y_offset = 0;
  const long long need = fused_im2col_ws_parts(dtype, m, taps, channels, &y_offset);
  if (workspace_bytes < need)
    return static_scratch
               ? fail(BEVK_ERR_INVALID,
                      "%s: this shape needs %lld bytes of scratch; the library's static "
                      "scratch holds %lld (use the workspace entry point)",
                      fn, need, (long long)workspace_bytes)
               : fail(BEVK_ERR_INVALID, "%s: workspace of %lld bytes, %lld needed", fn,
                      (long long)workspace_bytes, need);
  if (!data_im || !w_off || !b_off || !data_col || (!static_scratch && !workspace))
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  if (static_scratch) {
    if (int rc = device_scratch(fn, &workspace)) return rc;
  }
  const hipStream_t st = (hipStream_t)stream;
  void *packed = workspace;
  float *y = reinterpret_cast<float *>(static_cast<char *>(workspace) + y_offset);
  // 1. offset-conv weight [3T][T][C] -> the fused kernel's layout. The fp32 layout
  //    [3T][T * C] is w_off as given: no pass. (Half types: reading w_off unpacked, 32 rows
  //    of 32 bytes per load, measured 3 us slower at res4 than packing it first.)
  const void *w_conv = w_off;
  if (dtype != BEVK_F32) {
    if (int rc = hip_status(bevk::launch_dcn_pack_weight(dtype, w_off, 3 * taps, channels,
                                                         taps, packed, st, /*src_tc=*/true),
                            fn))
      return rc;
    w_conv = packed;
  }
  // 2. y = offset conv without bias, fp32 accumulation, fp32 output (matrix cores)
  if (int rc = hip_status(bevk::launch_dcn_fused_nhwc(dtype, g, 3 * taps, data_im, nullptr,
                                                      bevk::kGeoRegular, nullptr, w_conv,
                                                      nullptr, y, st),
                          fn))
    return rc;
  // 3. sigmoid, bias and the deformable gather into the columns
  return hip_status(bevk::launch_im2col_nhwc_yf32(dtype, g, data_im, y, b_off, data_col, st),
                    fn);
}

int bevk_modulated_deformable_fused_im2col_nhwc(
    int dtype, const void *data_im, const void *w_off, const float *b_off, int batch_size,
    int channels, int height_im, int width_im, int height_col, int width_col, int kernel_h,
    int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w, int dilation_h,
    int dilation_w, int deformable_group, void *workspace, int64_t workspace_bytes,
    void *data_col, void *stream) {
  return fused_im2col_run("modulated_deformable_fused_im2col_nhwc", false, dtype, data_im,
                          w_off, b_off, batch_size, channels, height_im, width_im, height_col,
                          width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                          dilation_h, dilation_w, deformable_group, workspace,
                          workspace_bytes, data_col, stream);
}

int bevk_modulated_deformable_fused_im2col_nhwc_noalloc(
    int dtype, const void *data_im, const void *w_off, const float *b_off, int batch_size,
    int channels, int height_im, int width_im, int height_col, int width_col, int kernel_h,
    int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w, int dilation_h,
    int dilation_w, int deformable_group, void *data_col, void *stream) {
  return fused_im2col_run("modulated_deformable_fused_im2col_nhwc_noalloc", true, dtype, data_im,
                          w_off, b_off, batch_size, channels, height_im, width_im, height_col,
                          width_col, kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w,
                          dilation_h, dilation_w, deformable_group, nullptr,
                          (int64_t)kNoAllocScratchBytes, data_col, stream);
}

int64_t bevk_dcn_packed_weight_bytes(int dtype, int channels_out, int kernel_h, int kernel_w,
                                      int channels) {
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16) return -1;
  if (channels_out < 0 || kernel_h <= 0 || kernel_w <= 0 || channels < 0) return -1;
  return bevk::dcn_packed_weight_elems(dtype, channels_out, kernel_h * kernel_w * channels) *
         dtype_size(dtype);
}

int bevk_dcn_pack_weight(int dtype, const void *weight, int channels_out, int kernel_h,
                         int kernel_w, int channels, void *packed, void *stream) {
  const char *fn = "dcn_pack_weight";
  g_last_error.clear();
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  if (channels_out < 0 || kernel_h <= 0 || kernel_w <= 0 || channels < 0)
    return fail(BEVK_ERR_INVALID, "%s: invalid weight shape", fn);
  const long long bytes = bevk::dcn_packed_weight_elems(dtype, channels_out,
                                                        kernel_h * kernel_w * channels) *
                          dtype_size(dtype);
  if (bytes == 0) return ok();
  if (bytes > kMaxBufferBytes)
    return fail(BEVK_ERR_INVALID, "%s: weight too large for 32-bit buffer offsets", fn);
  if (!weight || !packed) return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_dcn_pack_weight(dtype, weight, channels_out, channels,
                                                 kernel_h * kernel_w, packed,
                                                 (hipStream_t)stream),
                    fn);
}

int bevk_transpose(int dtype, const void *src, void *dst, int batch, int rows, int cols,
                   void *stream) {
  const char *fn = "transpose";
  g_last_error.clear();
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  if (batch < 0 || rows < 0 || cols < 0)
    return fail(BEVK_ERR_INVALID, "%s: negative size", fn);
  if (batch == 0 || rows == 0 || cols == 0) return ok();
  if (batch > 65535 || (rows + 63) / 64 > 65535 || (cols + 63) / 64 > (1 << 30))
    return fail(BEVK_ERR_INVALID, "%s: shape exceeds the launch grid", fn);
  if (!src || !dst) return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_transpose(dtype_size(dtype), src, dst, batch, rows, cols,
                                           (hipStream_t)stream),
                    fn);
}

int bevk_dcn_fused_fwd_nhwc(int dtype, const void *data_im, const void *data_offset,
                            int offset_last_dim, const void *data_mask, const void *weight_packed,
                            const void *bias, int batch_size, int channels, int height_im,
                            int width_im, int height_col, int width_col, int channels_out,
                            int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h,
                            int stride_w, int dilation_h, int dilation_w, void *out,
                            void *stream) {
  const char *fn = "dcn_fused_fwd_nhwc";
  g_last_error.clear();
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_geom(fn, g)) return rc;
  if (channels_out < 0) return fail(BEVK_ERR_INVALID, "%s: negative channels_out", fn);
  const int taps = kernel_h * kernel_w;
  if (offset_last_dim != 2 * taps && offset_last_dim != 3 * taps)
    return fail(BEVK_ERR_INVALID, "%s: offset last dim must be 2T (%d) or 3T (%d), got %d", fn,
                2 * taps, 3 * taps, offset_last_dim);
  const bool fused_y = offset_last_dim == 3 * taps;
  const long long m = (long long)batch_size * height_col * width_col;
  if (m * channels_out == 0) return ok();
  const int vec = 16 / dtype_size(dtype);
  if (channels <= 0 || channels % vec != 0)
    return fail(BEVK_ERR_UNSUPPORTED,
                "%s: channels (%d) must be a positive multiple of %d for '%s'", fn, channels,
                vec, dtype_name(dtype));
  if ((long long)batch_size * height_im * width_im * channels * dtype_size(dtype) >
          kMaxBufferBytes ||
      (long long)taps * channels * channels_out * dtype_size(dtype) > kMaxBufferBytes ||
      m >= (1LL << 30))
    return fail(BEVK_ERR_INVALID, "%s: problem too large for 32-bit buffer offsets", fn);
  if (bevk::dcn_packed_weight_elems(dtype, channels_out, taps * channels) * dtype_size(dtype) >
      kMaxBufferBytes)
    return fail(BEVK_ERR_INVALID, "%s: weight too large for 32-bit buffer offsets", fn);
  if (!data_im || !data_offset || (!fused_y && !data_mask) || !weight_packed || !out)
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_dcn_fused_nhwc(dtype, g, channels_out, data_im, data_offset,
                                                fused_y ? bevk::kGeoY : bevk::kGeoMask,
                                                data_mask, weight_packed, bias, out,
                                                (hipStream_t)stream),
                    fn);
}

// Shared checks of the offset-conv entry points (dg == 1, fused-kernel dtypes, channel
// vectors, 32-bit buffer offsets). Returns 0 or the failure code.
static int check_offset_conv(const char *fn, int dtype, const bevk::DcnGeom &g) {
  if (dtype != BEVK_F32 && dtype != BEVK_F16 && dtype != BEVK_BF16)
    return fail(BEVK_ERR_UNSUPPORTED, "\"%s\" not implemented for '%s'", fn, dtype_name(dtype));
  if (int rc = check_geom(fn, g)) return rc;
  const int taps = g.kernel_h * g.kernel_w;
  if (dtype != BEVK_F32 && taps > 9)
    return fail(BEVK_ERR_UNSUPPORTED,
                "%s: kernels of more than 9 taps are fp32-only for the offset conv", fn);
  const int vec = 16 / dtype_size(dtype);
  if (g.channels <= 0 || g.channels % vec != 0)
    return fail(BEVK_ERR_UNSUPPORTED,
                "%s: channels (%d) must be a positive multiple of %d for '%s'", fn, g.channels,
                vec, dtype_name(dtype));
  const long long m = (long long)g.batch * g.height_col * g.width_col;
  if ((long long)g.batch * g.height * g.width * g.channels * dtype_size(dtype) >
          kMaxBufferBytes ||
      m >= (1LL << 30))
    return fail(BEVK_ERR_INVALID, "%s: problem too large for 32-bit buffer offsets", fn);
  return 0;
}

int bevk_dcn_offset_conv_nhwc(int dtype, const void *data_im, const void *w_off_packed,
                              const float *b_off, int batch_size, int channels, int height_im,
                              int width_im, int height_col, int width_col, int kernel_h,
                              int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
                              int dilation_h, int dilation_w, float *y, void *stream) {
  const char *fn = "dcn_offset_conv_nhwc";
  g_last_error.clear();
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_offset_conv(fn, dtype, g)) return rc;
  const int taps = kernel_h * kernel_w;
  if ((long long)batch_size * height_col * width_col == 0) return ok();
  if (!data_im || !w_off_packed || !y) return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  return hip_status(bevk::launch_dcn_fused_nhwc(dtype, g, 3 * taps, data_im, nullptr,
                                                bevk::kGeoRegular, nullptr, w_off_packed, b_off,
                                                y, (hipStream_t)stream),
                    fn);
}

int bevk_dcn_mega_fwd_nhwc(int dtype, const void *data_im, const void *w_off_packed,
                           const float *b_off, const void *weight_packed, const void *bias,
                           int batch_size, int channels, int height_im, int width_im,
                           int height_col, int width_col, int channels_out, int kernel_h,
                           int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
                           int dilation_h, int dilation_w, int act_relu, float *y, void *out,
                           void *stream) {
  const char *fn = "dcn_mega_fwd_nhwc";
  g_last_error.clear();
  const bevk::DcnGeom g =
      make_geom(batch_size, channels, height_im, width_im, height_col, width_col, kernel_h,
                kernel_w, pad_h, pad_w, stride_h, stride_w, dilation_h, dilation_w, 1);
  if (int rc = check_offset_conv(fn, dtype, g)) return rc;
  if (channels_out < 0) return fail(BEVK_ERR_INVALID, "%s: negative channels_out", fn);
  const int taps = kernel_h * kernel_w;
  const long long m = (long long)batch_size * height_col * width_col;
  if (m == 0) return ok();
  if ((long long)taps * channels * channels_out * dtype_size(dtype) > kMaxBufferBytes ||
      bevk::dcn_packed_weight_elems(dtype, channels_out, taps * channels) * dtype_size(dtype) >
          kMaxBufferBytes)
    return fail(BEVK_ERR_INVALID, "%s: weight too large for 32-bit buffer offsets", fn);
  if (!data_im || !w_off_packed || !y || (channels_out > 0 && (!weight_packed || !out)))
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  const hipStream_t st = (hipStream_t)stream;
  if (channels_out > 0 && bevk::dcn_mega_supported(dtype, g, channels_out, out))
    return hip_status(bevk::launch_dcn_mega(dtype, g, channels_out, data_im, w_off_packed, b_off,
                                            weight_packed, bias, act_relu != 0, y, out, st),
                      fn);
  // Other shapes: the offset conv (with its bias) into y, then the fused kernel reading y.
  if (int rc = hip_status(bevk::launch_dcn_fused_nhwc(dtype, g, 3 * taps, data_im, nullptr,
                                                      bevk::kGeoRegular, nullptr, w_off_packed,
                                                      b_off, y, st),
                          fn))
    return rc;
  if (channels_out == 0) return ok();
  return hip_status(bevk::launch_dcn_fused_nhwc(dtype, g, channels_out, data_im, y,
                                                bevk::kGeoYF32, nullptr, weight_packed, bias,
                                                out, st, nullptr, act_relu != 0),
                    fn);
}

int bevk_msda_forward(int dtype, const void *value, const int64_t *spatial_shapes,
                      const int64_t *level_start_index, const void *sampling_loc,
                      const void *attn_weight, int batch, int spatial_size, int num_heads,
                      int channels, int num_levels, int num_query, int num_point,
                      int im2col_step, int force_generic, void *output, void *stream) {
  const char *fn = "msda_forward";
  g_last_error.clear();
  if (!valid_dtype(dtype)) return fail(BEVK_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (batch < 0 || spatial_size < 0 || num_heads < 0 || channels < 0 || num_levels < 0 ||
      num_query < 0 || num_point < 0)
    return fail(BEVK_ERR_INVALID, "%s: negative size", fn);
  if (im2col_step <= 0) return fail(BEVK_ERR_INVALID, "%s: im2col_step must be positive", fn);
  // binding_musa.mu:308-309
  const int step = batch < im2col_step ? batch : im2col_step;
  if (step > 0 && batch % step != 0)
    return fail(BEVK_ERR_INVALID, "batch must divide im2col_step");
  const long long n = (long long)batch * num_query * num_heads * channels;
  if (n == 0) return ok();
  if (!value || !spatial_shapes || !level_start_index || !sampling_loc || !attn_weight ||
      !output)
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  bevk::MsdaArgs a;
  a.value = value; a.spatial_shapes = spatial_shapes; a.level_start_index = level_start_index;
  a.sampling_loc = sampling_loc; a.attn_weight = attn_weight; a.output = output;
  a.batch = batch; a.spatial_size = spatial_size; a.num_heads = num_heads;
  a.channels = channels; a.num_levels = num_levels; a.num_query = num_query;
  a.num_point = num_point;
  return hip_status(
      bevk::launch_msda_forward(dtype, a, force_generic != 0, (hipStream_t)stream), fn);
}

int64_t bevk_msda_backward_workspace_bytes(int dtype, int batch, int spatial_size,
                                           int num_heads, int channels, int num_levels,
                                           int num_query, int num_point) {
  if (!valid_dtype(dtype) || batch < 0 || spatial_size < 0 || num_heads < 0 || channels < 0 ||
      num_levels < 0 || num_query < 0 || num_point < 0)
    return -1;
  return bevk::msda_backward_workspace_bytes(dtype, batch, spatial_size, num_heads, channels,
                                             num_levels, num_query, num_point);
}

int bevk_msda_backward(int dtype, const void *value, const int64_t *spatial_shapes,
                       const int64_t *level_start_index, const void *sampling_loc,
                       const void *attn_weight, const void *grad_output, int64_t go_stride_b,
                       int64_t go_stride_q, int64_t go_stride_h, int64_t go_stride_c,
                       int batch, int spatial_size, int num_heads, int channels,
                       int num_levels, int num_query, int num_point, int im2col_step,
                       int force_generic_col2im, void *grad_value, void *grad_sampling_loc,
                       void *grad_attn_weight, void *workspace, int64_t workspace_bytes,
                       void *stream) {
  const char *fn = "msda_backward";
  g_last_error.clear();
  if (!valid_dtype(dtype)) return fail(BEVK_ERR_INVALID, "%s: unknown dtype code %d", fn, dtype);
  if (batch < 0 || spatial_size < 0 || num_heads < 0 || channels < 0 || num_levels < 0 ||
      num_query < 0 || num_point < 0)
    return fail(BEVK_ERR_INVALID, "%s: negative size", fn);
  if (im2col_step <= 0) return fail(BEVK_ERR_INVALID, "%s: im2col_step must be positive", fn);
  // binding_musa.mu:438-439
  const int step = batch < im2col_step ? batch : im2col_step;
  if (step > 0 && batch % step != 0)
    return fail(BEVK_ERR_INVALID, "batch must divide im2col_step");
  const int64_t value_elems = (int64_t)batch * spatial_size * num_heads * channels;
  const int64_t need = bevk::msda_backward_workspace_min(dtype, value_elems);
  if (workspace_bytes < need)
    return fail(BEVK_ERR_INVALID, "%s: workspace of %lld bytes, %lld needed", fn,
                (long long)workspace_bytes, (long long)need);
  const long long units = (long long)batch * num_query * num_heads;
  // 16-bit grad_value is fully written (narrowed from the cleared accumulator) even when
  // there are no queries; with no values there is nothing to write at all
  if (value_elems == 0 || (units == 0 && need == 0)) return ok();
  if (channels == 0) return ok();
  if (!value || !spatial_shapes || !level_start_index || !grad_value ||
      (units > 0 && (!sampling_loc || !attn_weight || !grad_output || !grad_sampling_loc ||
                     !grad_attn_weight)) ||
      (need > 0 && !workspace))
    return fail(BEVK_ERR_INVALID, "%s: null tensor pointer", fn);
  if (units * 64 >= (1LL << 42))
    return fail(BEVK_ERR_INVALID, "%s: problem too large", fn);
  bevk::MsdaBwdArgs a;
  a.f.value = value; a.f.spatial_shapes = spatial_shapes;
  a.f.level_start_index = level_start_index; a.f.sampling_loc = sampling_loc;
  a.f.attn_weight = attn_weight; a.f.output = nullptr;
  a.f.batch = batch; a.f.spatial_size = spatial_size; a.f.num_heads = num_heads;
  a.f.channels = channels; a.f.num_levels = num_levels; a.f.num_query = num_query;
  a.f.num_point = num_point;
  a.grad_output = grad_output;
  a.go_stride[0] = go_stride_b; a.go_stride[1] = go_stride_q;
  a.go_stride[2] = go_stride_h; a.go_stride[3] = go_stride_c;
  a.grad_value = grad_value; a.grad_loc = grad_sampling_loc; a.grad_attn = grad_attn_weight;
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  return hip_status(
      bevk::launch_msda_backward(dtype, a, force_generic_col2im != 0, (hipStream_t)stream), fn);
}

}  // extern "C"
