// DCNv2 backward on gfx950: the column-to-image steps (NHWC and NCHW).
//
// Semantics (naotic/bev-kernels dcn_fused_nhwc_kernel.cuh:642-711, the per-element
// kernel the reference's NHWC backward runs by default): for every column element
// dcol[m, t*C + c] of output pixel m = (b, oh, ow) and tap t,
//   (h, w)   = (oh*sh - ph + i*dh + dy, ow*sw - pw + j*dw + dx), corners clipped one by one
//   dS       = dcol * mask
//   gX[b, corner, c] += dS * bilinear weight of the corner        (fp32 atomics)
//   gOff[m, 2t]     = sum_c dS * d(bilinear)/dh
//   gOff[m, 2t + 1] = sum_c dS * d(bilinear)/dw
//   gMask[m, t]     = sum_c dcol * bilinear, times s(1 - s) when the mask is the sigmoid s
//                     of a raw offset-conv output y (3T form: the sigmoid backward is folded in)
// A corner outside the image contributes nothing (the reference checks each corner; there
// is no separate -1 / H gate in the backward).
//
// Mapping: LPP = min(64, next power of two >= C) lanes own one (m, t) pair; lane li takes
// channels li, li + LPP, ..., so each gX atomic instruction adds LPP consecutive floats
// (fp32 atomics are issued per cache line: one lane holding 4 or 8 consecutive channels
// made them 4-9x slower). The three reductions over channels meet in a shuffle butterfly
// and one lane writes them (no atomics, no pre-zeroing for gOff / gMask). gX needs
// atomics: several pairs touch one input pixel.
#include "bevk_common.h"
#include "bevk_launch.h"

#include <hip/amd_detail/amd_hip_unsafe_atomics.h>
#include <type_traits>

namespace bevk {
namespace {

constexpr int kBlock = 256;

template <typename T, bool FUSED_Y>
__global__ void __launch_bounds__(kBlock) col2im_nhwc_kernel(
    const T *__restrict__ dcol, const T *__restrict__ im, const T *__restrict__ offset,
    const T *__restrict__ mask, const DcnGeom g, int lpp_log2, float *__restrict__ gx,
    float *__restrict__ goff, float *__restrict__ gmask) {
  const int T_ = g.kernel_h * g.kernel_w;
  const int HoWo = g.height_col * g.width_col;
  const int b = blockIdx.y;
  const int pair = (blockIdx.x * kBlock + threadIdx.x) >> lpp_log2;
  const int LPP = 1 << lpp_log2;
  const int li = threadIdx.x & (LPP - 1);
  // Lanes past the last pair still take part in the butterfly below; they do no work.
  const bool live = pair < HoWo * T_;
  const int pc = live ? pair : 0;
  // Quotients by the runtime sizes from a float reciprocal, corrected by one step (the
  // launch keeps every quotient below 2^22, where the estimate is off by at most one).
  auto qdiv = [](int a, int d) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
    const int r = a - q * d;
    return q + (r >= d) - (r < 0);
  };
  const int sp = qdiv(pc, T_), t = pc - sp * T_;
  const int oh = qdiv(sp, g.width_col), ow = sp - oh * g.width_col;
  const int i = qdiv(t, g.kernel_w), j = t - i * g.kernel_w;
  const int m = b * HoWo + sp;  // 32-bit indices: the launch checks the tensor sizes

  float dy, dx, mk;
  if constexpr (FUSED_Y) {
    const T *yp = offset + m * 3 * T_;
    dy = (float)yp[2 * t];
    dx = (float)yp[2 * t + 1];
    mk = sigmoid_f32((float)yp[2 * T_ + t]);
  } else {
    dy = (float)offset[m * 2 * T_ + 2 * t];
    dx = (float)offset[m * 2 * T_ + 2 * t + 1];
    mk = (float)mask[m * T_ + t];
  }
  const float h = (float)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
  const float w = (float)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
  const float fh = floorf(h), fw = floorf(w);
  const float lh = h - fh, lw = w - fw, hh = 1.f - lh, hw = 1.f - lw;
  // Corner validity, one by one. Clamp before converting so that far-away samples
  // cannot overflow int.
  const float fhc = fminf(fmaxf(fh, -2.f), (float)g.height);
  const float fwc = fminf(fmaxf(fw, -2.f), (float)g.width);
  const int hl = (int)fhc, wl = (int)fwc;
  const bool in_h0 = hl >= 0 && hl < g.height, in_h1 = hl + 1 >= 0 && hl + 1 < g.height;
  const bool in_w0 = wl >= 0 && wl < g.width, in_w1 = wl + 1 >= 0 && wl + 1 < g.width;
  // finite coordinates only: NaN / inf offsets touch nothing
  const bool fin = live && fh == fhc && fw == fwc;
  const bool c1 = fin && in_h0 && in_w0, c2 = fin && in_h0 && in_w1;
  const bool c3 = fin && in_h1 && in_w0, c4 = fin && in_h1 && in_w1;
  const float w1 = hh * hw, w2 = hh * lw, w3 = lh * hw, w4 = lh * lw;

  const int C = g.channels;
  const int64_t img = (int64_t)b * g.height * g.width;
  const int64_t p1 = (img + (int64_t)hl * g.width + wl) * C;
  const int64_t p2 = p1 + C, p3 = p1 + (int64_t)g.width * C, p4 = p3 + C;
  const T *drow = dcol + (m * T_ + t) * C;
  const bool coord = goff != nullptr;  // gX alone needs no image reads
  float ah = 0.f, aw = 0.f, am = 0.f;
  if (live) {
    // lane li takes channels li, li + LPP, ...: every load and every atomic below covers
    // LPP consecutive elements (fp32 atomics run several times slower when the lanes of
    // one instruction are spread over more cache lines)
#pragma unroll 4
    for (int c = li; c < C; c += LPP) {
      const float dc = (float)drow[c], ds = dc * mk;
      float x1 = 0.f, x2 = 0.f, x3 = 0.f, x4 = 0.f;
      if (coord) {
        if (c1) x1 = (float)im[p1 + c];
        if (c2) x2 = (float)im[p2 + c];
        if (c3) x3 = (float)im[p3 + c];
        if (c4) x4 = (float)im[p4 + c];
        ah += ds * (-hw * x1 - lw * x2 + hw * x3 + lw * x4);
        aw += ds * (-hh * x1 + hh * x2 - lh * x3 + lh * x4);
        am += dc * (w1 * x1 + w2 * x2 + w3 * x3 + w4 * x4);
      }
      if (gx != nullptr) {
        if (c1) unsafeAtomicAdd(gx + p1 + c, ds * w1);
        if (c2) unsafeAtomicAdd(gx + p2 + c, ds * w2);
        if (c3) unsafeAtomicAdd(gx + p3 + c, ds * w3);
        if (c4) unsafeAtomicAdd(gx + p4 + c, ds * w4);
      }
    }
  }
  for (int s = 1; s < LPP; s <<= 1) {
    ah += __shfl_xor(ah, s);
    aw += __shfl_xor(aw, s);
    am += __shfl_xor(am, s);
  }
  if (live && li == 0 && goff != nullptr) {
    goff[m * 2 * T_ + 2 * t] = ah;
    goff[m * 2 * T_ + 2 * t + 1] = aw;
    gmask[m * T_ + t] = FUSED_Y ? am * mk * (1.f - mk) : am;
  }
}

// ---------------------------------------------------------------------------
// NCHW (any deformable_group): columns [C*T, B*Ho*Wo] (row c*T + t). Semantics of the
// reference's NCHW backward (modulated_deform_conv_cuda_kernel.cuh:62-131, :257-339,
// :509-620, :824-937): a sample with h <= -1, w <= -1, h >= H or w >= W contributes nothing
// (to grad_im, grad_offset and grad_mask); inside, corners are checked one by one.
//   grad_im[b, c, corner]          += col * mask * corner weight        (atomics, dtype T)
//   grad_offset[b, g*2T + 2t(+1)]   = sum_c col * mask * d(bilinear)/dh (dw)   (written)
//   grad_mask[b, g*T + t]           = sum_c col * bilinear                   (written)
// One thread per (b, group, tap, output position); it walks the group's channels, so the
// channel sums need no reduction and consecutive threads read consecutive column entries.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void atomic_add_elem(float *p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_add_elem(double *p, double v) { unsafeAtomicAdd(p, v); }
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef short short2v __attribute__((ext_vector_type(2)));
// 16-bit types: a packed add on the aligned pair with -0.0 into the neighbour, the exact
// additive identity (x + -0.0 == x for every x, -0.0 and +0.0 included), so the
// neighbour keeps its bits. The entry point requires a 4-byte-aligned grad_im, so the
// first element has no neighbour before the buffer.
constexpr short kNegZero16 = (short)0x8000;  // -0.0 in fp16 and in bf16
__device__ __forceinline__ void atomic_add_elem(f16 *p, float v) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  half2v *pair = reinterpret_cast<half2v *>(a & ~(uintptr_t)3);
  const f16 h = (f16)v, nz = __builtin_bit_cast(f16, kNegZero16);
  half2v d = (a & 2) ? half2v{nz, h} : half2v{h, nz};
  __builtin_amdgcn_global_atomic_fadd_v2f16(pair, d);
}
__device__ __forceinline__ void atomic_add_elem(bf16 *p, float v) {
  const uintptr_t a = reinterpret_cast<uintptr_t>(p);
  short2v *pair = reinterpret_cast<short2v *>(a & ~(uintptr_t)3);
  const short b = __builtin_bit_cast(short, (bf16)v);
  short2v d = (a & 2) ? short2v{kNegZero16, b} : short2v{b, kNegZero16};
  __builtin_amdgcn_global_atomic_fadd_v2bf16(pair, d);
}

template <typename T>
__global__ void __launch_bounds__(kBlock) col2im_nchw_kernel(
    const T *__restrict__ col, const T *__restrict__ im, const T *__restrict__ offset,
    const T *__restrict__ mask, const DcnGeom g, T *__restrict__ grad_im,
    T *__restrict__ grad_offset, T *__restrict__ grad_mask) {
  using A = typename Acc<T>::type;
  const int T_ = g.kernel_h * g.kernel_w;
  const int HoWo = g.height_col * g.width_col;
  const int64_t n = (int64_t)g.batch * g.deformable_group * T_ * HoWo;
  const int64_t idx = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (idx >= n) return;
  const int sp = (int)(idx % HoWo);
  int64_t r = idx / HoWo;
  const int t = (int)(r % T_);
  r /= T_;
  const int grp = (int)(r % g.deformable_group);
  const int b = (int)(r / g.deformable_group);
  const int oh = sp / g.width_col, ow = sp - oh * g.width_col;
  const int i = t / g.kernel_w, j = t - i * g.kernel_w;
  const int cpg = g.channels / g.deformable_group;

  const int64_t og = ((int64_t)b * g.deformable_group + grp) * T_;  // (b, group) tap base
  const A dy = (A)offset[((og + t) * 2) * HoWo + sp];
  const A dx = (A)offset[((og + t) * 2 + 1) * HoWo + sp];
  const A mk = (A)mask[(og + t) * HoWo + sp];
  const A h = (A)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
  const A w = (A)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
  A gh = 0, gw = 0, gm = 0;
  if (h > (A)-1 && w > (A)-1 && h < (A)g.height && w < (A)g.width) {
    const A fh = floor(h), fw = floor(w);
    const int hl = (int)fh, wl = (int)fw;
    const A lh = h - fh, lw = w - fw, hh = (A)1 - lh, hw = (A)1 - lw;
    const bool c1 = hl >= 0 && wl >= 0, c2 = hl >= 0 && wl + 1 <= g.width - 1;
    const bool c3 = hl + 1 <= g.height - 1 && wl >= 0;
    const bool c4 = hl + 1 <= g.height - 1 && wl + 1 <= g.width - 1;
    const A w1 = hh * hw, w2 = hh * lw, w3 = lh * hw, w4 = lh * lw;
    const int64_t plane = (int64_t)g.height * g.width;
    const int64_t q1 = (int64_t)hl * g.width + wl, q2 = q1 + 1, q3 = q1 + g.width, q4 = q3 + 1;
    const int64_t bhw = (int64_t)g.batch * HoWo;
    const int c0 = grp * cpg;
    for (int c = c0; c < c0 + cpg; ++c) {
      const A dc = (A)col[((int64_t)c * T_ + t) * bhw + (int64_t)b * HoWo + sp];
      const A ds = dc * mk;
      const int64_t pb = ((int64_t)b * g.channels + c) * plane;
      if (grad_im != nullptr) {
        if (c1) atomic_add_elem(grad_im + pb + q1, ds * w1);
        if (c2) atomic_add_elem(grad_im + pb + q2, ds * w2);
        if (c3) atomic_add_elem(grad_im + pb + q3, ds * w3);
        if (c4) atomic_add_elem(grad_im + pb + q4, ds * w4);
      }
      if (grad_offset != nullptr) {
        const A x1 = c1 ? (A)im[pb + q1] : (A)0, x2 = c2 ? (A)im[pb + q2] : (A)0;
        const A x3 = c3 ? (A)im[pb + q3] : (A)0, x4 = c4 ? (A)im[pb + q4] : (A)0;
        gh += ds * (-hw * x1 - lw * x2 + hw * x3 + lw * x4);
        gw += ds * (-hh * x1 + hh * x2 - lh * x3 + lh * x4);
        gm += dc * (w1 * x1 + w2 * x2 + w3 * x3 + w4 * x4);
      }
    }
  }
  if (grad_offset != nullptr) {
    grad_offset[((og + t) * 2) * HoWo + sp] = (T)gh;
    grad_offset[((og + t) * 2 + 1) * HoWo + sp] = (T)gw;
    grad_mask[(og + t) * HoWo + sp] = (T)gm;
  }
}

template <typename T>
hipError_t launch_nchw_t(const DcnGeom &g, const void *col, const void *im, const void *off,
                         const void *msk, void *grad_im, void *grad_offset, void *grad_mask,
                         hipStream_t stream) {
  const int64_t n = (int64_t)g.batch * g.deformable_group * g.kernel_h * g.kernel_w *
                    g.height_col * g.width_col;
  hipLaunchKernelGGL(col2im_nchw_kernel<T>, dim3((unsigned)((n + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, stream, static_cast<const T *>(col),
                     static_cast<const T *>(im), static_cast<const T *>(off),
                     static_cast<const T *>(msk), g, static_cast<T *>(grad_im),
                     static_cast<T *>(grad_offset), static_cast<T *>(grad_mask));
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// NHWC grad_offset / grad_mask alone, 16-byte vectors: lane li of a pair's LPP lanes takes
// the VEC = 16 / sizeof(T) consecutive channels at li*VEC (then + LPP*VEC), so one dcol
// load and four corner loads move 16 bytes per lane; LPP = min(8, next power of two >=
// C / VEC): eight pairs share a wave, so the per-pair geometry (the bulk of the VALU work)
// is repeated on 8 lanes, not 64 (measured at res4: 8 lanes 51 / 107 us fp16 / fp32,
// 64 lanes 68 / 142 us, 4 lanes 60 / 142 us). Corners outside the
// image read zeros through the buffer path (their offset is set past the end of the
// image), so there are no branches around the loads. The gradients are formed from the
// four corner dot products once per (pixel, tap) after a shuffle butterfly.
// ---------------------------------------------------------------------------
template <typename T, bool FUSED_Y>
__global__ void __launch_bounds__(kBlock) col2im_coord_nhwc_vec_kernel(
    const T *__restrict__ dcol, const T *__restrict__ im, const T *__restrict__ offset,
    const T *__restrict__ mask, const DcnGeom g, int lpp_log2, uint32_t im_bytes,
    float *__restrict__ goff, float *__restrict__ gmask) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr uint32_t kPast = 0x80000000u;  // >= im_bytes: loads there return zeros
  const int T_ = g.kernel_h * g.kernel_w;
  const int HoWo = g.height_col * g.width_col;
  const int b = blockIdx.y;
  const int pair = (blockIdx.x * kBlock + threadIdx.x) >> lpp_log2;
  const int LPP = 1 << lpp_log2;
  const int li = threadIdx.x & (LPP - 1);
  const bool live = pair < HoWo * T_;
  const int pc = live ? pair : 0;
  // Quotients by the runtime sizes from a float reciprocal, corrected by one step (the
  // launch keeps every quotient below 2^22, where the estimate is off by at most one).
  auto qdiv = [](int a, int d) {
    int q = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
    const int r = a - q * d;
    return q + (r >= d) - (r < 0);
  };
  const int sp = qdiv(pc, T_), t = pc - sp * T_;
  const int oh = qdiv(sp, g.width_col), ow = sp - oh * g.width_col;
  const int i = qdiv(t, g.kernel_w), j = t - i * g.kernel_w;
  const int m = b * HoWo + sp;  // 32-bit indices: the launch checks the tensor sizes

  float dy, dx, mk;
  if constexpr (FUSED_Y) {
    const T *yp = offset + m * 3 * T_;
    dy = (float)yp[2 * t];
    dx = (float)yp[2 * t + 1];
    mk = sigmoid_f32((float)yp[2 * T_ + t]);
  } else {
    dy = (float)offset[m * 2 * T_ + 2 * t];
    dx = (float)offset[m * 2 * T_ + 2 * t + 1];
    mk = (float)mask[m * T_ + t];
  }
  const float h = (float)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
  const float w = (float)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
  const float fh = floorf(h), fw = floorf(w);
  const float lh = h - fh, lw = w - fw, hh = 1.f - lh, hw = 1.f - lw;
  const float fhc = fminf(fmaxf(fh, -2.f), (float)g.height);
  const float fwc = fminf(fmaxf(fw, -2.f), (float)g.width);
  const int hl = (int)fhc, wl = (int)fwc;
  const bool in_h0 = hl >= 0 && hl < g.height, in_h1 = hl + 1 >= 0 && hl + 1 < g.height;
  const bool in_w0 = wl >= 0 && wl < g.width, in_w1 = wl + 1 >= 0 && wl + 1 < g.width;
  const bool fin = live && fh == fhc && fw == fwc;
  const int C = g.channels;
  const int img = b * g.height * g.width;
  const uint32_t eb = (uint32_t)sizeof(T);
  const uint32_t e1 = (uint32_t)((img + hl * g.width + wl) * C) * eb;  // corner 1, bytes
  const uint32_t rowb = (uint32_t)(g.width * C) * eb, colb = (uint32_t)C * eb;
  const uint32_t o1 = (fin && in_h0 && in_w0) ? e1 : kPast;
  const uint32_t o2 = (fin && in_h0 && in_w1) ? e1 + colb : kPast;
  const uint32_t o3 = (fin && in_h1 && in_w0) ? e1 + rowb : kPast;
  const uint32_t o4 = (fin && in_h1 && in_w1) ? e1 + rowb + colb : kPast;
  const float w1 = hh * hw, w2 = hh * lw, w3 = lh * hw, w4 = lh * lw;
  const __amdgpu_buffer_rsrc_t rim = make_rsrc(im, im_bytes);
  const T *drow = dcol + (m * T_ + t) * C;
  // The three gradients are fixed combinations of the corner dot products
  // S_k = sum_c dcol[c] * x_k[c]; the lanes accumulate S_1..S_4 (two channels per
  // v_dot2 for the 16-bit types: exact products, fp32 sums) and lane 0 combines them.
  float s1 = 0.f, s2 = 0.f, s3 = 0.f, s4 = 0.f;
  if (live) {
    for (int c = li * VEC; c < C; c += LPP * VEC) {
      const Vec<T, VEC> dv = load_vec_nt<T, VEC>(drow + c);  // read once: keep x in L2
      const uint32_t cb = (uint32_t)c * eb;
      const Vec<T, VEC> v1 = buffer_load_vec<T, VEC>(rim, o1 + cb);
      const Vec<T, VEC> v2 = buffer_load_vec<T, VEC>(rim, o2 + cb);
      const Vec<T, VEC> v3 = buffer_load_vec<T, VEC>(rim, o3 + cb);
      const Vec<T, VEC> v4 = buffer_load_vec<T, VEC>(rim, o4 + cb);
      if constexpr (sizeof(T) == 2) {
        using P2 = T __attribute__((ext_vector_type(2)));
        struct Pairs { P2 p[VEC / 2]; };
        const Pairs d = __builtin_bit_cast(Pairs, dv), p1 = __builtin_bit_cast(Pairs, v1);
        const Pairs p2 = __builtin_bit_cast(Pairs, v2), p3 = __builtin_bit_cast(Pairs, v3);
        const Pairs p4 = __builtin_bit_cast(Pairs, v4);
#pragma unroll
        for (int e = 0; e < VEC / 2; ++e) {
          if constexpr (std::is_same_v<T, f16>) {
            s1 = __builtin_amdgcn_fdot2(d.p[e], p1.p[e], s1, false);
            s2 = __builtin_amdgcn_fdot2(d.p[e], p2.p[e], s2, false);
            s3 = __builtin_amdgcn_fdot2(d.p[e], p3.p[e], s3, false);
            s4 = __builtin_amdgcn_fdot2(d.p[e], p4.p[e], s4, false);
          } else {
            s1 = __builtin_amdgcn_fdot2_f32_bf16(d.p[e], p1.p[e], s1, false);
            s2 = __builtin_amdgcn_fdot2_f32_bf16(d.p[e], p2.p[e], s2, false);
            s3 = __builtin_amdgcn_fdot2_f32_bf16(d.p[e], p3.p[e], s3, false);
            s4 = __builtin_amdgcn_fdot2_f32_bf16(d.p[e], p4.p[e], s4, false);
          }
        }
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          const float dc = (float)dv.v[e];
          s1 = fmaf(dc, (float)v1.v[e], s1);
          s2 = fmaf(dc, (float)v2.v[e], s2);
          s3 = fmaf(dc, (float)v3.v[e], s3);
          s4 = fmaf(dc, (float)v4.v[e], s4);
        }
      }
    }
  }
  if (LPP >= 4) {
    // Packed reduction over the LPP lanes: the lower half keeps (S1, S2) and the upper
    // half (S3, S4), then each quarter keeps one of them and sums it over its lanes; lane
    // 0 reads the other three totals (log2(LPP) + 4 shuffles instead of 4 log2(LPP)).
    const int hf = LPP >> 1, qt = LPP >> 2;
    const bool up = li & hf;
    float a = up ? s3 : s1, c = up ? s4 : s2;
    a += __shfl_xor(up ? s1 : s3, hf, kWave);
    c += __shfl_xor(up ? s2 : s4, hf, kWave);
    const bool up2 = li & qt;
    float v = up2 ? c : a;
    v += __shfl_xor(up2 ? a : c, qt, kWave);
    for (int st = qt >> 1; st >= 1; st >>= 1) v += __shfl_xor(v, st, kWave);
    const int base = (threadIdx.x & (kWave - 1)) & ~(LPP - 1);
    s1 = v;
    s2 = __shfl(v, base + qt, kWave);
    s3 = __shfl(v, base + hf, kWave);
    s4 = __shfl(v, base + hf + qt, kWave);
  } else {
    for (int st = 1; st < LPP; st <<= 1) {
      s1 += __shfl_xor(s1, st, kWave);
      s2 += __shfl_xor(s2, st, kWave);
      s3 += __shfl_xor(s3, st, kWave);
      s4 += __shfl_xor(s4, st, kWave);
    }
  }
  if (live && li == 0) {
    goff[m * 2 * T_ + 2 * t] = mk * (hw * (s3 - s1) + lw * (s4 - s2));
    goff[m * 2 * T_ + 2 * t + 1] = mk * (hh * (s2 - s1) + lh * (s4 - s3));
    const float am = w1 * s1 + w2 * s2 + w3 * s3 + w4 * s4;
    gmask[m * T_ + t] = FUSED_Y ? am * mk * (1.f - mk) : am;
  }
}

// ---------------------------------------------------------------------------
// NHWC grad_x by output tile (dg == 1), without float atomics in LDS. A workgroup takes a
// TH x TW tile of output pixels of one image and 64*CPL channels:
//   1. every (pixel, tap) sample's valid bilinear corners become (dcol row, weight * mask)
//      pairs, binned by target input position: one bin per position of the tile's input
//      footprint (the rows / columns its taps reach, grown by kGbMargin pixels for the
//      offsets) plus one bin for corners beyond it. An integer LDS atomic per pair gives
//      its rank inside its bin;
//   2. an exclusive scan of the bin counts gives the bin starts, and every pair is stored
//      at start + rank (a counting sort);
//   3. each wave takes whole bins: lane l holds channels l, l+64, ... and sums the bin's
//      pairs in registers (weight times the dcol element), then adds the sum to grad_x
//      with one fp32 atomic per channel. Pairs of the far bin are added one by one.
// Each input element receives ~36 contributions from a tile (9 taps x 4 corners); they
// collapse to one global atomic, and LDS only ever sees integer atomics (one per pair,
// not per channel). Same per-corner semantics as col2im_nhwc_kernel: finite coordinates
// only, each corner checked against the image.
// ---------------------------------------------------------------------------
constexpr int kGbThreads = 512;
constexpr int kGbMargin = 8;
constexpr int kGbMaxPos = 1024;                               // footprint bins
constexpr int kGbMaxPairs = 2304;                             // pairs per tile (4 per sample)
constexpr int kGbSPT = (kGbMaxPairs / 4 + kGbThreads - 1) / kGbThreads;  // samples / thread

struct GbPair {
  uint32_t row;  // dcol row (m * T + t)
  float w;       // bilinear weight times the modulation
  int tgt;       // near pairs: bin; far pairs: target pixel y * W + x
};

struct GxBin {
  int th, tw;        // output tile
  int rh, rw;        // footprint rows / columns
  int tiles_x, ntile, chunks;
  int per_xcd;       // items per XCD (XCD-contiguous item ranges)
  uint32_t dcol_bytes;  // bytes of dcol (the buffer range of the pair loads)
};

// One pair's CPL channels through the buffer path: lane offset in a VGPR, the pair's
// byte offset in an SGPR.
template <typename T, int N>
__device__ __forceinline__ Vec<T, N> buffer_load_vec_s(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                       uint32_t soff) {
  constexpr int bytes = sizeof(T) * N;
  if constexpr (bytes == 16) {
    return __builtin_bit_cast(Vec<T, N>, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
  } else if constexpr (bytes == 8) {
    return __builtin_bit_cast(Vec<T, N>, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0));
  } else if constexpr (bytes == 4) {
    return __builtin_bit_cast(Vec<T, N>, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
  } else {
    static_assert(bytes == 2, "unsupported vector width");
    return __builtin_bit_cast(Vec<T, N>, __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, 0));
  }
}

template <typename T, bool FUSED_Y, int CPL>
__global__ void __launch_bounds__(kGbThreads) col2im_nhwc_gx_bin_kernel(
    const T *__restrict__ dcol, const T *__restrict__ offset, const T *__restrict__ mask,
    const DcnGeom g, const GxBin tl, float *__restrict__ gx) {
  __shared__ int bin_at[kGbMaxPos + kGbThreads / kWave + 2];  // counts, then bin starts
  __shared__ int wsum[kGbThreads / kWave];
  __shared__ GbPair list[kGbMaxPairs];
  __shared__ float xpose[kGbThreads / kWave][kWave * CPL];
  const int T_ = g.kernel_h * g.kernel_w;
  const int HoWo = g.height_col * g.width_col;
  const int C = g.channels;
  const int nitems = g.batch * tl.ntile * tl.chunks;
  const int item = (int)(blockIdx.x & 7) * tl.per_xcd + (int)(blockIdx.x >> 3);
  if (item >= nitems || (int)(blockIdx.x >> 3) >= tl.per_xcd) return;  // uniform
  const int chunk = item % tl.chunks;
  const int tile = (item / tl.chunks) % tl.ntile;
  const int b = item / (tl.chunks * tl.ntile);
  const int ty = tile / tl.tiles_x, tx = tile - ty * tl.tiles_x;
  const int oh0 = ty * tl.th, ow0 = tx * tl.tw;
  const int fy0 = oh0 * g.stride_h - g.pad_h - kGbMargin;
  const int fx0 = ow0 * g.stride_w - g.pad_w - kGbMargin;
  // Footprint position p goes to bin (p % 8) * P8 + p / 8, so that wave w's bins (the
  // positions p = w mod 8) are contiguous in the sorted list; bin nnb takes the corners
  // beyond the footprint.
  constexpr int kNW = kGbThreads / kWave;
  const int npos = tl.rh * tl.rw;
  const int P8 = (npos + kNW - 1) / kNW;
  const int nnb = P8 * kNW;
  const int nbins = nnb + 1;
  const int tid = threadIdx.x;
  for (int i = tid; i < nbins + 1; i += kGbThreads) bin_at[i] = 0;
  __syncthreads();

  // 1. Pairs and their ranks (registers: kGbSPT samples x 4 corners per thread).
  const int nsamp = tl.th * tl.tw * T_;
  int pbin[kGbSPT][4], prank[kGbSPT][4], ptgt[kGbSPT][4];
  float pw[kGbSPT][4];
  uint32_t prow[kGbSPT];
#pragma unroll
  for (int k = 0; k < kGbSPT; ++k) {
    const int s = tid + k * kGbThreads;
    const int pix = s / T_, t = s - (s / T_) * T_;
    const int oh = oh0 + pix / tl.tw, ow = ow0 + pix % tl.tw;
    const bool live = s < nsamp && oh < g.height_col && ow < g.width_col;
    const int m = b * HoWo + (live ? oh * g.width_col + ow : 0);
    const int tt = live ? t : 0;
    float dy = 0.f, dx = 0.f, mk = 0.f;
    if (live) {
      if constexpr (FUSED_Y) {
        const T *o = offset + (int64_t)m * 3 * T_;
        dy = (float)o[2 * tt];
        dx = (float)o[2 * tt + 1];
        mk = sigmoid_f32((float)o[2 * T_ + tt]);
      } else {
        dy = (float)offset[(int64_t)m * 2 * T_ + 2 * tt];
        dx = (float)offset[(int64_t)m * 2 * T_ + 2 * tt + 1];
        mk = (float)mask[(int64_t)m * T_ + tt];
      }
    }
    prow[k] = (uint32_t)m * (uint32_t)T_ + (uint32_t)tt;
    const int i = tt / g.kernel_w, j = tt - i * g.kernel_w;
    const float h = (float)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
    const float w = (float)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
    const float fh = floorf(h), fw = floorf(w);
    const float lh = h - fh, lw = w - fw, hh = 1.f - lh, hw = 1.f - lw;
    const float fhc = fminf(fmaxf(fh, -2.f), (float)g.height);
    const float fwc = fminf(fmaxf(fw, -2.f), (float)g.width);
    const int hl = (int)fhc, wl = (int)fwc;
    const bool fin = live && fh == fhc && fw == fwc;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int yy = hl + (q >> 1), xx = wl + (q & 1);
      const bool ok = fin && yy >= 0 && yy < g.height && xx >= 0 && xx < g.width;
      const int ry = yy - fy0, rx = xx - fx0;
      const bool in = (unsigned)ry < (unsigned)tl.rh && (unsigned)rx < (unsigned)tl.rw;
      const int pos = ry * tl.rw + rx;
      const int nb = (pos % kNW) * P8 + pos / kNW;
      pbin[k][q] = ok ? (in ? nb : nnb) : -1;
      pw[k][q] = ((q >> 1) ? lh : hh) * ((q & 1) ? lw : hw) * mk;
      ptgt[k][q] = in ? nb : yy * g.width + xx;
      prank[k][q] = ok ? atomicAdd(&bin_at[pbin[k][q]], 1) : 0;
    }
  }
  __syncthreads();

  // 2. Exclusive scan of the nbins counts: thread tid owns entries [tid*E, tid*E + E).
  {
    const int E = (nbins + kGbThreads - 1) / kGbThreads;
    const int e0 = min(tid * E, nbins), e1 = min(e0 + E, nbins);
    int local = 0;
    for (int e = e0; e < e1; ++e) local += bin_at[e];
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    int incl = local;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int v = __shfl_up(incl, d, kWave);
      if (lane >= d) incl += v;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int run = incl - local;
    for (int w2 = 0; w2 < wave; ++w2) run += wsum[w2];
    for (int e = e0; e < e1; ++e) {
      const int c = bin_at[e];
      bin_at[e] = run;
      run += c;
    }
    if (tid == kGbThreads - 1) {
      int tot = 0;
      for (int w2 = 0; w2 < kGbThreads / kWave; ++w2) tot += wsum[w2];
      bin_at[nbins] = tot;
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kGbSPT; ++k)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (pbin[k][q] >= 0) list[bin_at[pbin[k][q]] + prank[k][q]] = GbPair{prow[k], pw[k][q], ptgt[k][q]};
  __syncthreads();

  // 3. Sums per bin. Wave w streams through the pairs of its bins (positions p = w mod 8
  // in row order: the waves sweep the footprint together, so the four corner reads of a
  // sample's dcol row, a footprint row apart, stay close in time and hit L2) in groups of
  // kG pairs, one list entry per lane; each pair's dcol offset, weight and bin are then
  // taken into scalar registers (readlane), so a pair costs one buffer load (scalar
  // offset) and CPL FMAs. Lane l holds the CPL consecutive channels at l*CPL of the
  // workgroup's 64*CPL. When the bin changes, the finished sum goes through the wave's
  // LDS slot so that each grad_x atomic instruction adds 64 consecutive floats (fp32
  // atomics are issued per cache line).
  const int lane = tid & (kWave - 1), wave = tid / kWave;
  const int64_t img = (int64_t)b * g.height * g.width;
  const int cbase = chunk * (kWave * CPL);
  float *gxc = gx + cbase + lane;
  float *xp = xpose[wave];
  const int lo = bin_at[wave * P8], hi = bin_at[(wave + 1) * P8];
  if (lo < hi) {
    auto flush = [&](int bin, const float *acc) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int c = 0; c < CPL; ++c) xp[lane * CPL + c] = acc[c];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const int pos = (bin % P8) * kNW + bin / P8;
      const int y = fy0 + pos / tl.rw, x = fx0 + pos % tl.rw;
      float *dst = gxc + (img + (int64_t)y * g.width + x) * C;
#pragma unroll
      for (int c = 0; c < CPL; ++c) unsafeAtomicAdd(dst + c * kWave, xp[c * kWave + lane]);
    };
    const __amdgpu_buffer_rsrc_t rdc = make_rsrc(dcol + cbase, tl.dcol_bytes - (uint32_t)(cbase * sizeof(T)));
    const uint32_t vlane = (uint32_t)(lane * CPL * sizeof(T));
    const uint32_t row_bytes = (uint32_t)(C * sizeof(T));
    constexpr int kG = sizeof(T) * CPL <= 8 ? 16 : 8;  // pairs per group
    // Lanes u < kG (and their copies every kG lanes) hold the entries of the group at k0.
    auto entries = [&](int k0) { return list[min(k0 + (lane & (kG - 1)), hi - 1)]; };
    auto issue = [&](const GbPair &e, Vec<T, CPL> *v) {
      const uint32_t off = e.row * row_bytes;
#pragma unroll
      for (int u = 0; u < kG; ++u)
        v[u] = buffer_load_vec_s<T, CPL>(rdc, vlane, (uint32_t)__builtin_amdgcn_readlane((int)off, u));
    };
    int cur = __builtin_amdgcn_readfirstlane(list[lo].tgt);
    float acc[CPL];
#pragma unroll
    for (int c = 0; c < CPL; ++c) acc[c] = 0.f;
    auto consume = [&](int k0, const GbPair &e, const Vec<T, CPL> *v) {
      const int ew = __builtin_bit_cast(int, e.w);
#pragma unroll
      for (int u = 0; u < kG; ++u) {
        if (k0 + u < hi) {
          const int t = __builtin_amdgcn_readlane(e.tgt, u);
          if (t != cur) {
            flush(cur, acc);
#pragma unroll
            for (int c = 0; c < CPL; ++c) acc[c] = 0.f;
            cur = t;
          }
          const float w = __builtin_bit_cast(float, __builtin_amdgcn_readlane(ew, u));
#pragma unroll
          for (int c = 0; c < CPL; ++c) acc[c] += w * (float)v[u].v[c];
        }
      }
    };
    // Two value buffers in turn (no register copies of loaded values, which would wait
    // for the loads): the group after next is in flight while a group is summed.
    Vec<T, CPL> va[kG], vb[kG];
    GbPair ea = entries(lo);
    issue(ea, va);
    for (int k0 = lo; k0 < hi; k0 += 2 * kG) {
      const GbPair eb = entries(k0 + kG);
      issue(eb, vb);
      consume(k0, ea, va);
      ea = entries(k0 + 2 * kG);
      issue(ea, va);
      consume(k0 + kG, eb, vb);
    }
    flush(cur, acc);
  }
  // Far bin: pairs spread over the waves, one pair at a time (lane l: channels l + 64c).
  const T *dcs = dcol + cbase + lane;
  for (int k = bin_at[nnb] + wave; k < bin_at[nbins]; k += kNW) {
    const GbPair e = list[k];
    float *dst = gxc + (img + e.tgt) * C;
#pragma unroll
    for (int c = 0; c < CPL; ++c)
      unsafeAtomicAdd(dst + c * kWave, e.w * (float)dcs[(int64_t)e.row * C + c * kWave]);
  }
}

// Tile plan for the binned grad_x kernel; false when C is not a multiple of 64 or a tile
// of the smallest size does not fit the LDS bins / pair list.
bool gx_bin_plan(const DcnGeom &g, int cpl, int elem_bytes, GxBin &tl) {
  const int T_ = g.kernel_h * g.kernel_w;
  if (g.deformable_group != 1 || g.channels <= 0 || g.channels % (kWave * cpl) != 0) return false;
  const int64_t dcol_bytes = (int64_t)g.batch * g.height_col * g.width_col * T_ * g.channels * elem_bytes;
  if (dcol_bytes >= ((int64_t)1 << 32)) return false;  // 32-bit buffer offsets
  tl.dcol_bytes = (uint32_t)dcol_bytes;
  int th = 8, tw = 8;
  auto extent = [&](int t, int s, int k, int d) {
    return (t - 1) * s + (k - 1) * d + 2 + 2 * kGbMargin;
  };
  auto fits = [&]() {
    return th * tw * T_ * 4 <= kGbMaxPairs &&
           extent(th, g.stride_h, g.kernel_h, g.dil_h) * extent(tw, g.stride_w, g.kernel_w, g.dil_w) <=
               kGbMaxPos;
  };
  while (!fits()) {
    if (th >= tw && th > 1) th /= 2;
    else if (tw > 1) tw /= 2;
    else return false;
  }
  tl.th = th;
  tl.tw = tw;
  tl.rh = extent(th, g.stride_h, g.kernel_h, g.dil_h);
  tl.rw = extent(tw, g.stride_w, g.kernel_w, g.dil_w);
  tl.tiles_x = (g.width_col + tw - 1) / tw;
  tl.ntile = tl.tiles_x * ((g.height_col + th - 1) / th);
  tl.chunks = g.channels / (kWave * cpl);
  const int64_t nitems = (int64_t)g.batch * tl.ntile * tl.chunks;
  if (nitems > (1 << 28)) return false;
  tl.per_xcd = (int)((nitems + 7) / 8);
  return true;
}

template <typename T, bool FY>
hipError_t launch_t(const DcnGeom &g, const void *dcol, const void *im, const void *off,
                    const void *msk, float *gx, float *goff, float *gmask, hipStream_t stream) {
  int lpp_log2 = 0;
  while (lpp_log2 < 6 && (1 << lpp_log2) < g.channels) ++lpp_log2;
  const int64_t pairs = (int64_t)g.height_col * g.width_col * g.kernel_h * g.kernel_w;
  const int64_t threads = pairs << lpp_log2;
  const dim3 grid((unsigned)((threads + kBlock - 1) / kBlock), g.batch);
  const T *dc = static_cast<const T *>(dcol), *of = static_cast<const T *>(off);
  const T *mk = static_cast<const T *>(msk), *xim = static_cast<const T *>(im);
  // grad_offset / grad_mask through the 16-byte kernel where rows are 16-byte aligned and
  // the image fits the 31-bit buffer offsets; grad_x then goes separately.
  constexpr int VEC = 16 / sizeof(T);
  const int64_t im_bytes = (int64_t)g.batch * g.height * g.width * g.channels * sizeof(T);
  const int64_t col_elems = (int64_t)g.batch * g.height_col * g.width_col *
                            g.kernel_h * g.kernel_w * g.channels;
  const bool vec = goff != nullptr && (sizeof(T) == 2 || sizeof(T) == 4) && g.channels % VEC == 0 &&
                   im_bytes < ((int64_t)1 << 31) && col_elems < ((int64_t)1 << 31) &&
                   (int64_t)g.batch * g.height_col * g.width_col * 3 * g.kernel_h * g.kernel_w <
                       ((int64_t)1 << 31) &&
                   (int64_t)g.height_col * g.width_col < ((int64_t)1 << 22) &&
                   reinterpret_cast<uintptr_t>(dcol) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(im) % 16 == 0;
  if (gx != nullptr) {
    // grad_x through the binned kernel where it applies, else through the per-sample
    // kernel (alone when the 16-byte kernel takes the coordinates).
    GxBin tl;
    const int cpl = g.channels % (4 * kWave) == 0 ? 4 : (g.channels % (2 * kWave) == 0 ? 2 : 1);
    if (g.channels % kWave == 0 && reinterpret_cast<uintptr_t>(dcol) % 16 == 0 &&
        gx_bin_plan(g, cpl, (int)sizeof(T), tl)) {
      const dim3 bgrid((unsigned)(tl.per_xcd * 8));
      if (cpl == 4)
        hipLaunchKernelGGL((col2im_nhwc_gx_bin_kernel<T, FY, 4>), bgrid, dim3(kGbThreads), 0, stream, dc, of, mk, g, tl, gx);
      else if (cpl == 2)
        hipLaunchKernelGGL((col2im_nhwc_gx_bin_kernel<T, FY, 2>), bgrid, dim3(kGbThreads), 0, stream, dc, of, mk, g, tl, gx);
      else
        hipLaunchKernelGGL((col2im_nhwc_gx_bin_kernel<T, FY, 1>), bgrid, dim3(kGbThreads), 0, stream, dc, of, mk, g, tl, gx);
      gx = nullptr;
    } else if (vec || goff == nullptr) {
      hipLaunchKernelGGL((col2im_nhwc_kernel<T, FY>), grid, dim3(kBlock), 0, stream, dc, xim,
                         of, mk, g, lpp_log2, gx, (float *)nullptr, (float *)nullptr);
      gx = nullptr;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || goff == nullptr) return e;
  }
  if (vec) {
    int vl2 = 0;
    while (vl2 < 3 && (1 << vl2) * VEC < g.channels) ++vl2;  // at most 8 lanes per pair
    const dim3 vgrid((unsigned)(((pairs << vl2) + kBlock - 1) / kBlock), g.batch);
    hipLaunchKernelGGL((col2im_coord_nhwc_vec_kernel<T, FY>), vgrid, dim3(kBlock), 0, stream, dc,
                       xim, of, mk, g, vl2, (uint32_t)im_bytes, goff, gmask);
  } else {
    hipLaunchKernelGGL((col2im_nhwc_kernel<T, FY>), grid, dim3(kBlock), 0, stream, dc, xim, of,
                       mk, g, lpp_log2, gx, goff, gmask);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_col2im_nchw(int dtype, const DcnGeom &g, const void *col, const void *im,
                              const void *off, const void *msk, void *grad_im,
                              void *grad_offset, void *grad_mask, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_nchw_t<float>(g, col, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    case 1: return launch_nchw_t<f16>(g, col, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    case 2: return launch_nchw_t<bf16>(g, col, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    case 3: return launch_nchw_t<double>(g, col, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_col2im_nhwc(int dtype, const DcnGeom &g, const void *dcol, const void *im,
                              const void *off, bool fused_y, const void *msk, float *grad_im,
                              float *grad_offset, float *grad_mask, hipStream_t stream) {
  switch (dtype) {
    case 0: return fused_y ? launch_t<float, true>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream)
                           : launch_t<float, false>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    case 1: return fused_y ? launch_t<f16, true>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream)
                           : launch_t<f16, false>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    case 2: return fused_y ? launch_t<bf16, true>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream)
                           : launch_t<bf16, false>(g, dcol, im, off, msk, grad_im, grad_offset, grad_mask, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
