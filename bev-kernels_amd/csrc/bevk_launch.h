// Internal launcher interface between the C ABI (binding.cpp) and the kernel
// translation units. Arguments are already validated by the caller; each launcher
// only enqueues work and returns the HIP status of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "bevk_common.h"

namespace bevk {

// Compute units of the current device (cached per device; 0 when the query fails).
int device_cus();

struct MsdaArgs {
  const void *value;
  const int64_t *spatial_shapes;
  const int64_t *level_start_index;
  const void *sampling_loc;
  const void *attn_weight;
  void *output;
  int batch, spatial_size, num_heads, channels, num_levels, num_query, num_point;
};

hipError_t launch_msda_forward(int dtype, const MsdaArgs &a, bool force_generic,
                               hipStream_t stream);

// MSDA backward: f holds the forward inputs (f.output unused).
struct MsdaBwdArgs {
  MsdaArgs f;
  const void *grad_output;
  int64_t go_stride[4];  // grad_output strides over (batch, query, head, channel), elements
  void *grad_value, *grad_loc, *grad_attn;
  void *workspace;       // fp32 accumulator for 16-bit dtypes, then the sorted path's buffers
  int64_t workspace_bytes;
};

// Bytes of fp32 accumulator the 16-bit backward needs at least (0 for f32 / f64).
int64_t msda_backward_workspace_min(int dtype, int64_t value_elems);
// Bytes that also hold the buffers of the sorted grad_value path (D = 32), which runs when
// the workspace is at least this large.
int64_t msda_backward_workspace_bytes(int dtype, int64_t batch, int64_t spatial_size,
                                      int64_t num_heads, int64_t channels, int64_t num_levels,
                                      int64_t num_query, int64_t num_point);
// force_generic: the per-unit atomic kernel for every level (no coarse split, no grid
// owner pass, no D = 32 kernel).
hipError_t launch_msda_backward(int dtype, const MsdaBwdArgs &a, bool force_generic,
                                hipStream_t stream);

struct DcnGeom {
  int batch, channels, height, width, height_col, width_col;
  int kernel_h, kernel_w, pad_h, pad_w, stride_h, stride_w, dil_h, dil_w;
  int deformable_group;
};

// NCHW modulated im2col; `tiled` picks the geometry-reuse kernel (im2col_opt).
hipError_t launch_im2col_nchw(int dtype, const DcnGeom &g, const void *data_im,
                              const void *data_offset, const void *data_mask,
                              void *data_col, bool tiled, hipStream_t stream);

// NHWC gather (dg == 1). fused_y: data_offset is the raw [.., 3T] offset-conv output.
hipError_t launch_im2col_nhwc(int dtype, const DcnGeom &g, const void *data_im,
                              const void *data_offset, bool fused_y, const void *data_mask,
                              void *data_col, hipStream_t stream);

// Fused NHWC implicit-GEMM forward (dg == 1). w_packed: layout of launch_dcn_pack_weight.
// geo (DcnGeo): kGeoMask / kGeoY read data_offset (and data_mask) in the input dtype;
// kGeoYF32 reads an fp32 y [M][3T] as data_offset and adds y_bias [3T] (fp32, may be
// null); kGeoRegular ignores data_offset / data_mask and writes fp32 `out`, with an fp32
// `bias`. relu: max(out, 0) in the epilogue (not for kGeoRegular).
hipError_t launch_dcn_fused_nhwc(int dtype, const DcnGeom &g, int channels_out,
                                 const void *data_im, const void *data_offset, int geo,
                                 const void *data_mask, const void *w_packed,
                                 const void *bias, void *out, hipStream_t stream,
                                 const float *y_bias = nullptr, bool relu = false);

// fp16 / bf16 implicit GEMM with the weight in MFMA-fragment blocks (<= 9 taps).
bool dcn_fused_h_supported(const DcnGeom &g);
hipError_t launch_dcn_fused_h(int dtype, const DcnGeom &g, int channels_out, const void *x,
                              const void *off, int geo, const void *msk,
                              const void *w_packed, const void *bias, void *out,
                              hipStream_t stream, const float *y_bias = nullptr,
                              bool relu = false);

// One-launch DCNv2 forward with the offset conv inside (fp16 / bf16 on the persistent
// kernel): y = conv(x, w_off) + b_off (fp32, kept in LDS and written to y_out), offsets
// y[:, :2T], mask sigmoid(y[:, 2T:]), then the deformable implicit GEMM (+ bias, relu).
// Returns false (and launches nothing) when the shape does not take the persistent
// kernel; the caller then runs the offset conv and launch_dcn_fused_nhwc (kGeoYF32).
bool dcn_mega_supported(int dtype, const DcnGeom &g, int channels_out, const void *out);
hipError_t launch_dcn_mega(int dtype, const DcnGeom &g, int channels_out, const void *x,
                           const void *w_off_packed, const float *b_off,
                           const void *w_packed, const void *bias, bool relu, float *y_out,
                           void *out, hipStream_t stream);

// Elements of the packed weight: fp32 Cout * K; half types ceil(Cout/32) * ceil(K/16) * 512.
int64_t dcn_packed_weight_elems(int dtype, int cout, int K);
// Weight [Cout][C][kh*kw] (module layout; [Cout][kh*kw][C] with src_tc) -> packed: fp32
// [Cout][kh*kw][C]; fp16 / bf16 MFMA-fragment blocks (block (n/32, k/16), lane
// (n%32) + 32*((k%16)/8), 8 consecutive k), k = t*C + c, zero outside [0, Cout) x [0, K).
hipError_t launch_dcn_pack_weight(int dtype, const void *weight, int cout, int C, int T,
                                  void *packed, hipStream_t stream, bool src_tc = false);

// dst[b][c][r] = src[b][r][c] for 2- or 4-byte elements (NCHW <-> NHWC).
hipError_t launch_transpose(int elem_bytes, const void *src, void *dst, int batch, int rows,
                            int cols, hipStream_t stream);

// NHWC gather whose offsets / pre-sigmoid mask come from an fp32 y [M][3T] plus an fp32
// bias [3T] (the fused front end: y is the offset conv without its bias).
hipError_t launch_im2col_nhwc_yf32(int dtype, const DcnGeom &g, const void *data_im,
                                   const float *y, const float *y_bias, void *data_col,
                                   hipStream_t stream);

// NCHW column-to-image backward (any dg), gradients in the input dtype: grad_im accumulated
// with atomics (caller zeroes it; skipped when null), grad_offset / grad_mask written
// (skipped when grad_offset is null).
hipError_t launch_col2im_nchw(int dtype, const DcnGeom &g, const void *col, const void *im,
                              const void *off, const void *msk, void *grad_im,
                              void *grad_offset, void *grad_mask, hipStream_t stream);

// NHWC column-to-image backward (dg == 1): grad_im [B,H,W,C] fp32 accumulated with atomics
// (caller zeroes it; skipped when null), grad_offset [M][2T] and grad_mask [M][T] fp32
// written (skipped when grad_offset is null). fused_y: offsets / pre-sigmoid mask from
// y [M][3T] and grad_mask is the gradient of the pre-sigmoid value.
hipError_t launch_col2im_nhwc(int dtype, const DcnGeom &g, const void *dcol, const void *im,
                              const void *off, bool fused_y, const void *msk, float *grad_im,
                              float *grad_offset, float *grad_mask, hipStream_t stream);

}  // namespace bevk
