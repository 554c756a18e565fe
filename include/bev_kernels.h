/*
 * bev_kernels.h — C ABI of libbevk.so, the MI355X (gfx950) implementation of the
 * BEVFormer deformable-conv (DCNv2) and multi-scale deformable attention (MSDA)
 * operators: forward, backward and the layout / weight-packing helpers.
 *
 * Conventions shared by every entry point:
 *   - All data pointers are DEVICE pointers to dense, contiguous (row-major) buffers.
 *     The caller allocates every input and output; the library allocates nothing
 *     that outlives a call.
 *   - `dtype` selects the element type of the floating-point buffers (bevk_dtype).
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Work is
 *     enqueued asynchronously; nothing synchronises the host.
 *   - Return value: 0 on success, otherwise a bevk_status code; the message for the
 *     last failure on the calling thread is returned by bevk_last_error().
 *   - Arguments are validated before any device work is enqueued; a rejected call
 *     leaves every output untouched.
 *
 * Each entry point names the reference interface it replaces (naotic/bev-kernels,
 * file:line). The reference exposes these through pybind11 on at::Tensor; here the
 * same argument order is kept with tensors lowered to (pointer, dtype) pairs.
 */
#ifndef BEV_KERNELS_H_
#define BEV_KERNELS_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  BEVK_F32 = 0,
  BEVK_F16 = 1,
  BEVK_BF16 = 2,
  BEVK_F64 = 3
} bevk_dtype;

typedef enum {
  BEVK_OK = 0,
  BEVK_ERR_INVALID = 1,     /* argument validation failed (RuntimeError in Python) */
  BEVK_ERR_UNSUPPORTED = 2, /* dtype / shape combination not implemented           */
  BEVK_ERR_HIP = 3          /* HIP runtime reported an error at launch              */
} bevk_status;

/* Message describing the most recent failed call on this thread ("" if none). */
const char *bevk_last_error(void);

/* Library version string, e.g. "bevk 0.1.0 gfx950". */
const char *bevk_version(void);

/* ------------------------------------------------------------------------- */
/* DCNv2, NCHW layout                                                         */
/* ------------------------------------------------------------------------- */

/* Modulated deformable im2col, NCHW.
 *   data_im     [B, C, H, W]
 *   data_offset [B, dg*2*kh*kw, Ho, Wo]   (dy, dx) interleaved per tap
 *   data_mask   [B, dg*kh*kw, Ho, Wo]
 *   data_col    [C*kh*kw, B, Ho, Wo]      row = c*kh*kw + (i*kw + j); fully written
 * Replaces binding.cpp:5-11 / :142-144 (modulated_deformable_im2col_cuda, launcher
 * modulated_deform_conv_cuda.cu:4-30). dtypes: F32, F64, F16, BF16. */
int bevk_modulated_deformable_im2col(
    int dtype, const void *data_im, const void *data_offset, const void *data_mask,
    int batch_size, int channels, int height_im, int width_im, int height_col,
    int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h,
    int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *data_col, void *stream);

/* Same contract as bevk_modulated_deformable_im2col; the tiled kernel that the
 * reference's module forward uses.
 * Replaces binding.cpp:21-27 / :149-151 (modulated_deformable_im2col_opt_cuda,
 * launcher modulated_deform_conv_cuda.cu:62-115). */
int bevk_modulated_deformable_im2col_opt(
    int dtype, const void *data_im, const void *data_offset, const void *data_mask,
    int batch_size, int channels, int height_im, int width_im, int height_col,
    int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h,
    int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *data_col, void *stream);

/* ------------------------------------------------------------------------- */
/* DCNv2, NHWC layout (deformable_group == 1)                                 */
/* ------------------------------------------------------------------------- */

/* Deformable gather into columns, NHWC.
 *   data_im     [B, H, W, C]
 *   data_offset [B, Ho, Wo, offset_last_dim]. offset_last_dim == 2T: offsets
 *               (dy, dx per tap) and data_mask [B, Ho, Wo, T] holds the mask.
 *               offset_last_dim == 3T: the raw offset-conv output y; offsets are
 *               y[..., :2T] and mask = sigmoid(y[..., 2T:]); data_mask is ignored.
 *   data_col    [B*Ho*Wo, T*C], k = t*C + c; fully written.
 * Replaces binding.cpp:64-70 / :164-166 (modulated_deformable_im2col_nhwc_cuda,
 * launcher dcn_fused_nhwc_cuda.cu:27-87, fused-y rule at :54). */
int bevk_modulated_deformable_im2col_nhwc(
    int dtype, const void *data_im, const void *data_offset, int offset_last_dim,
    const void *data_mask, int batch_size, int channels, int height_im, int width_im,
    int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *data_col, void *stream);

/* NCHW backward, column to image (any deformable_group):
 *   data_col     [C*kh*kw, B*Ho*Wo] gradient of the columns (row c*T + t), dtype
 *   data_im      [B, C, H, W] (may be NULL when grad_offset is NULL)
 *   data_offset  [B, dg*2T, Ho, Wo], data_mask [B, dg*T, Ho, Wo]
 *   grad_im      [B, C, H, W] dtype, ACCUMULATED with atomics (zero it first), or NULL. For
 *                F16 / BF16 the adds are packed pairs with -0.0 (the exact identity) added
 *                to the neighbour element, so grad_im must be 4-byte aligned
 *                (BEVK_ERR_INVALID otherwise) and, with an odd element count, the 2 bytes
 *                after it must be addressable (they keep their bits).
 *   grad_offset  [B, dg*2T, Ho, Wo] and grad_mask [B, dg*T, Ho, Wo] dtype, written, or NULL
 * Replaces binding.cpp:13-19, :29-58 (modulated_deformable_col2im[_opt|_smem]_cuda and
 * modulated_deformable_col2im_coord[_opt]_cuda; modulated_deform_conv_cuda_kernel.cuh:
 * 62-131, :195-339, :509-937). A sample outside (-1, H) x (-1, W) contributes nothing.
 * dtypes F32, F16, BF16, F64. */
int bevk_modulated_deformable_col2im_nchw(
    int dtype, const void *data_col, const void *data_im, const void *data_offset,
    const void *data_mask, int batch_size, int channels, int height_im, int width_im,
    int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    void *grad_im, void *grad_offset, void *grad_mask, void *stream);

/* NHWC backward, column to image (dg == 1):
 *   dcol         [B*Ho*Wo, T*C] gradient of the columns, dtype
 *   data_im, data_offset, offset_last_dim, data_mask: as bevk_modulated_deformable_im2col_nhwc
 *                (data_im may be NULL when grad_offset is NULL: grad_im needs no image)
 *   grad_im      [B, H, W, C] fp32, ACCUMULATED with atomics (zero it first), or NULL
 *   grad_offset  [B*Ho*Wo, 2T] fp32, written, or NULL (then grad_mask NULL too)
 *   grad_mask    [B*Ho*Wo, T] fp32, written: the gradient of the mask, or of the
 *                pre-sigmoid mask in the 3T form (sigmoid backward folded in)
 * Replaces binding.cpp:80-86 modulated_deformable_col2im_nhwc_cuda and its variants
 * (col2im_coord_nhwc, gradx_smem / gradx_gather, col2im_fused_smem, col2im_perelem[_smem],
 * binding.cpp:88-140; per-element semantics of dcn_fused_nhwc_kernel.cuh:642-711).
 * dtypes F32, F16, BF16. */
int bevk_modulated_deformable_col2im_nhwc(
    int dtype, const void *dcol, const void *data_im, const void *data_offset,
    int offset_last_dim, const void *data_mask, int batch_size, int channels, int height_im,
    int width_im, int height_col, int width_col, int kernel_h, int kernel_w, int pad_h, int pad_w,
    int stride_h, int stride_w, int dilation_h, int dilation_w, int deformable_group,
    float *grad_im, float *grad_offset, float *grad_mask, void *stream);

/* Workspace bytes bevk_modulated_deformable_fused_im2col_nhwc needs (-1 on bad
 * arguments): the packed offset-conv weight and the fp32 offset-conv output [M][3T]. */
int64_t bevk_dcn_fused_im2col_nhwc_workspace_bytes(int dtype, int batch_size, int channels,
                                                   int height_col, int width_col, int kernel_h,
                                                   int kernel_w);

/* Fused NHWC front end: offset conv + sigmoid + deformable gather.
 *   data_im   [B, H, W, C]
 *   w_off     [3T, T, C] (= torch weight [3T, C, kh, kw].permute(0, 2, 3, 1)), dtype
 *   b_off     [3T] fp32
 *   data_col  [B*Ho*Wo, T*C], fully written
 * y = conv(x, w_off) + b_off is accumulated in fp32 and kept in fp32 (matrix cores, with the
 * same stride / padding / dilation as the deformable taps); offsets = y[:, :2T] ((dy, dx) per
 * tap), mask = sigmoid(y[:, 2T:3T]); then the NHWC gather. `workspace` (device memory of at
 * least bevk_dcn_fused_im2col_nhwc_workspace_bytes) holds y and, for F16 / BF16, the packed
 * w_off (F32 reads w_off as given; the size is the same for every dtype).
 * Replaces binding.cpp:72-78 modulated_deformable_fused_im2col_nhwc_cuda
 * (dcn_fused_nhwc_cuda.cu:92-126, kernel dcn_fused_nhwc_kernel.cuh:211-303). dg == 1.
 * dtypes F32 (any kernel size), F16 / BF16 (at most 9 taps); C a multiple of 16 bytes'
 * worth of elements. */
int bevk_modulated_deformable_fused_im2col_nhwc(
    int dtype, const void *data_im, const void *w_off, const float *b_off, int batch_size,
    int channels, int height_im, int width_im, int height_col, int width_col, int kernel_h,
    int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w, int dilation_h,
    int dilation_w, int deformable_group, void *workspace, int64_t workspace_bytes,
    void *data_col, void *stream);

/* The fused NHWC front end above without a workspace argument: it allocates nothing
 * (no hipMalloc / hipFree, no allocating library call) and keeps the packed offset-conv
 * weight and the fp32 offset-conv output in a 16 MiB static device array of the library
 * (one copy per GPU, held until the process ends). No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops).
 * Shapes whose scratch need (bevk_dcn_fused_im2col_nhwc_workspace_bytes) exceeds 16 MiB
 * return BEVK_ERR_INVALID before any device work. Calls that overlap on one GPU share the
 * array and race; everything in it is written before it is read, so nothing carries over
 * between calls. Arguments and results as bevk_modulated_deformable_fused_im2col_nhwc. */
int bevk_modulated_deformable_fused_im2col_nhwc_noalloc(
    int dtype, const void *data_im, const void *w_off, const float *b_off, int batch_size,
    int channels, int height_im, int width_im, int height_col, int width_col, int kernel_h,
    int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w, int dilation_h,
    int dilation_w, int deformable_group, void *data_col, void *stream);

/* Bytes of the packed weight that bevk_dcn_fused_fwd_nhwc consumes for this shape
 * (-1 for an unsupported dtype). */
int64_t bevk_dcn_packed_weight_bytes(int dtype, int channels_out, int kernel_h, int kernel_w,
                                     int channels);

/* Repacks a module weight [Cout, C, kh, kw] (the layout of ModulatedDeformConv2d.weight)
 * into the fused kernel's layout, into `packed` (bevk_dcn_packed_weight_bytes bytes):
 *   F32:       [Cout, kh, kw, C]
 *   F16, BF16: MFMA-fragment blocks: block (n/32, k/16) of 64 lanes x 8 elements, lane
 *              (n%32) + 32*((k%16)/8), k = (i*kw + j)*C + c; zero padded to whole blocks.
 * The reference flattens its weight on every call (weight.permute(2,3,1,0), e.g.
 * fused_tl.py:500-510, dcn_split_nhwc.py:143); the Python operators pack on every call
 * too, a caller with a fixed weight may pack once. */
int bevk_dcn_pack_weight(int dtype, const void *weight, int channels_out, int kernel_h,
                         int kernel_w, int channels, void *packed, void *stream);

/* Layout change: dst[b][c][r] = src[b][r][c] over a [batch, rows, cols] source, i.e.
 * NCHW -> NHWC with rows = C, cols = H*W, and back with rows = H*W, cols = C. No
 * counterpart in the reference, whose NCHW module path feeds NCHW kernels; here the NCHW
 * module (modulated_deform_conv.py:331-403 interface) runs the NHWC fused kernel and
 * changes layout on the way in and out. dtypes: F16, BF16, F32; bit-exact copy. */
int bevk_transpose(int dtype, const void *src, void *dst, int batch, int rows, int cols,
                   void *stream);

/* Fused NHWC DCNv2 forward: bilinear x mask taps are produced straight into LDS and
 * multiplied on the matrix cores; no column buffer touches HBM.
 *   data_im       [B, H, W, C]
 *   data_offset   [B, Ho, Wo, offset_last_dim] with the same 2T / 3T rule as above
 *   data_mask     [B, Ho, Wo, T] (ignored in the 3T form)
 *   weight_packed the output of bevk_dcn_pack_weight
 *   bias          [Cout] in dtype, or NULL
 *   out           [B, Ho, Wo, Cout]; fully written. fp32 accumulation, one rounding.
 * C must be a multiple of 16 bytes' worth of elements (8 for F16/BF16, 4 for F32).
 * Computes fused_tl.fused_dcn_forward_nhwc (fused_tl.py:513-556, algorithm of the
 * T.gemm kernel at :42-139) and the forward of DCNSplitNHWCFunction
 * (dcn_split_nhwc.py:158-228) after its offset conv. dtypes: F16, BF16, F32. */
int bevk_dcn_fused_fwd_nhwc(
    int dtype, const void *data_im, const void *data_offset, int offset_last_dim,
    const void *data_mask, const void *weight_packed, const void *bias, int batch_size,
    int channels, int height_im, int width_im, int height_col, int width_col,
    int channels_out, int kernel_h, int kernel_w, int pad_h, int pad_w, int stride_h,
    int stride_w, int dilation_h, int dilation_w, void *out, void *stream);

/* Offset conv of the NHWC front end on the matrix cores:
 *   data_im       [B, H, W, C]
 *   w_off_packed  bevk_dcn_pack_weight of the offset-conv weight [3T, C, kh, kw]
 *                 (channels_out = 3T)
 *   b_off         [3T] fp32, or NULL
 *   y             [B*Ho*Wo, 3T] fp32, written: conv(x, w_off) + b_off, accumulated in fp32
 * Offsets are y[:, :2T] ((dy, dx) per tap) and the pre-sigmoid mask y[:, 2T:].
 * Replaces fused_tl.offset_conv_forward_nhwc's kernel (fused_tl.py:419-470: fp32
 * accumulation, fp32 output, bias added in fp32). dg == 1. dtypes F32 (any kernel size),
 * F16 / BF16 (at most 9 taps); C a multiple of 16 bytes' worth of elements. */
int bevk_dcn_offset_conv_nhwc(int dtype, const void *data_im, const void *w_off_packed,
                              const float *b_off, int batch_size, int channels, int height_im,
                              int width_im, int height_col, int width_col, int kernel_h,
                              int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
                              int dilation_h, int dilation_w, float *y, void *stream);

/* Whole DCNv2 forward with the offset conv inside (the reference's single-kernel
 * fused_dcn_mega_forward_nhwc, fused_tl.py:565-766, and the forward of
 * DCNSplitNHWCFunction with its FrozenBN + ReLU epilogue, dcn_split_nhwc.py:158-204):
 *   y = conv(x, w_off) + b_off in fp32 (as bevk_dcn_offset_conv_nhwc; written to y,
 *   [B*Ho*Wo, 3T] fp32, which the backward needs), offsets y[:, :2T], mask
 *   sigmoid(y[:, 2T:]), then out = deformable conv (+ bias) as bevk_dcn_fused_fwd_nhwc,
 *   with max(out, 0) when act_relu != 0.
 *   weight_packed / bias / out: as bevk_dcn_fused_fwd_nhwc (channels_out may be 0: y only).
 * F16 / BF16 shapes that take the persistent kernels with one column half (C % 64 == 0,
 * 128 < Cout <= 256, Cout % 8 == 0, any row count) run as ONE launch: y stays in LDS for
 * the gather and never returns from HBM. Other shapes (Cout > 256 among them, where one
 * launch would compute the offset conv once per column half) run the offset conv and then
 * the fused kernel reading y. dtypes F32, F16, BF16; dg == 1. */
int bevk_dcn_mega_fwd_nhwc(int dtype, const void *data_im, const void *w_off_packed,
                           const float *b_off, const void *weight_packed, const void *bias,
                           int batch_size, int channels, int height_im, int width_im,
                           int height_col, int width_col, int channels_out, int kernel_h,
                           int kernel_w, int pad_h, int pad_w, int stride_h, int stride_w,
                           int dilation_h, int dilation_w, int act_relu, float *y, void *out,
                           void *stream);

/* ------------------------------------------------------------------------- */
/* Multi-scale deformable attention                                            */
/* ------------------------------------------------------------------------- */

/* MSDA forward.
 *   value              [B, spatial_size, num_heads, channels]
 *   spatial_shapes     [num_levels, 2] int64 (H_l, W_l), device memory
 *   level_start_index  [num_levels]    int64, device memory
 *   sampling_loc       [B, num_query, num_heads, num_levels, num_point, 2] (x, y) in [0,1]
 *   attn_weight        [B, num_query, num_heads, num_levels, num_point]
 *   output             [B, num_query, num_heads*channels]; fully written (samples
 *                      outside a level contribute zero).
 * im2col_step keeps the reference's contract (batch % min(batch, step) == 0); the
 * whole batch is processed by one launch. force_generic selects the
 * thread-per-output-element kernel.
 * Replaces _msda_opt2_musa.forward (binding_musa.mu:286-412, :546-549).
 * dtypes: F32, F16, BF16 (fp32 accumulation), F64. */
int bevk_msda_forward(
    int dtype, const void *value, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_loc, const void *attn_weight,
    int batch, int spatial_size, int num_heads, int channels, int num_levels,
    int num_query, int num_point, int im2col_step, int force_generic, void *output,
    void *stream);

/* Bytes of workspace for bevk_msda_backward, -1 for an unknown dtype or a negative size.
 * F16/BF16 need at least an fp32 accumulator of batch*spatial_size*num_heads*channels
 * elements (the reference allocates it inside its fp16 backward, binding_musa.mu:456-463;
 * here the caller owns it); F32/F64 need none. With channels == 32 the value returned
 * also holds the buffers of the sorted grad_value path (for every sample, up to two
 * 12-byte records, one per image row of its valid corners, bucketed by position), which
 * bevk_msda_backward takes whenever
 * the workspace it is given is at least this large; a smaller workspace (at least the
 * accumulator) runs the atomic kernels instead. */
int64_t bevk_msda_backward_workspace_bytes(int dtype, int batch, int spatial_size,
                                           int num_heads, int channels, int num_levels,
                                           int num_query, int num_point);

/* MSDA backward.
 *   value, spatial_shapes, level_start_index, sampling_loc, attn_weight: as the forward.
 *   grad_output        [B, num_query, num_heads*channels]; go_stride_{b,q,h,c} are its
 *                      element strides over (batch, query, head, channel) (the
 *                      reference reads a strided grad_output too).
 *   grad_value         [B, spatial_size, num_heads, channels]. F32/F64: gradients are
 *                      ADDED to what it holds (the caller zeroes it, as
 *                      ms_deform_attn_backward in dispatch.py:36-69 does). F16/BF16: the
 *                      gradient is accumulated in the fp32 workspace, which is cleared
 *                      here, and then written over grad_value.
 *   grad_sampling_loc  [B, num_query, num_heads, num_levels, num_point, 2]; written.
 *   grad_attn_weight   [B, num_query, num_heads, num_levels, num_point]; written.
 *   workspace          bevk_msda_backward_workspace_bytes(...) bytes, device memory.
 * im2col_step keeps the reference's contract. force_generic_col2im != 0 runs the
 * per-(batch, query, head) kernel alone, adding every level's grad_value with atomics
 * (the reference's generic col2im, binding_musa.mu:459); otherwise the sorted grad_value
 * path (D = 32, full workspace), then the grid-query owner pass or the D = 32 kernel with
 * the coarse-level sort (smaller workspaces) are used where they apply.
 * spatial_shapes / level_start_index must describe value (lsi[l] + H_l * W_l <=
 * spatial_size), as in the reference; they are read on the device only.
 * Replaces _msda_opt2_musa.backward (binding_musa.mu:414-543, :550-556).
 * dtypes: F32, F16, BF16 (fp32 arithmetic and accumulation), F64. */
int bevk_msda_backward(
    int dtype, const void *value, const int64_t *spatial_shapes,
    const int64_t *level_start_index, const void *sampling_loc, const void *attn_weight,
    const void *grad_output, int64_t go_stride_b, int64_t go_stride_q, int64_t go_stride_h,
    int64_t go_stride_c, int batch, int spatial_size, int num_heads, int channels,
    int num_levels, int num_query, int num_point, int im2col_step, int force_generic_col2im,
    void *grad_value, void *grad_sampling_loc, void *grad_attn_weight, void *workspace,
    int64_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* BEV_KERNELS_H_ */
