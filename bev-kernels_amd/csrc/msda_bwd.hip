// Multi-scale deformable attention, backward, for gfx950.
//
// Semantics (naotic/bev-kernels ms_deform_attn_kernels.cuh:427-490, :638-790;
// binding_musa.mu:414-543): for every (b, q, head, level, point) sample at
//   h_im = loc_y * H_l - 0.5, w_im = loc_x * W_l - 0.5, inside (-1, H_l) x (-1, W_l),
// with top = grad_output[b, q, head*D + c] and a = attn[b, q, head, l, p]:
//   grad_value[b, corner, head, c] += corner weight * top * a      (atomic adds)
//   grad_loc[..., 0] = W_l * sum_c top * a * d(bilinear)/dw_im     (written)
//   grad_loc[..., 1] = H_l * sum_c top * a * d(bilinear)/dh_im     (written)
//   grad_attn        = sum_c top * bilinear                        (written)
// A corner outside the level contributes nothing (each corner checked on its own); a
// sample outside the (-1, H_l) x (-1, W_l) window writes zeros.
//
// Mapping: G = min(64, next power of two >= D) consecutive lanes of one wave own a
// (b, q, head) unit; lane j takes channels j, j+G, ... A corner row of D channels is then
// one coalesced access, for the value loads and for the atomics, and the channel sums of
// a sample meet in a butterfly over the G lanes. The unit walks its L*P samples in
// order, so its grad_loc / grad_attn rows are written front to back.
//
// grad_value is fp32 for f32/f16/bf16 inputs and fp64 for f64: 16-bit callers pass an
// fp32 workspace that is cleared here, accumulated, and narrowed into grad_value at the
// end (binding_musa.mu:456-510 does the same for fp16).
#include "bevk_common.h"
#include "bevk_launch.h"

#include <hip/amd_detail/amd_hip_unsafe_atomics.h>

namespace bevk {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ void atomic_acc(float *p, float v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void atomic_acc(double *p, double v) { unsafeAtomicAdd(p, v); }

struct BwdParams {
  const int64_t *shapes, *lsi;
  int64_t go_sb, go_sq, go_sh, go_sc;  // grad_output strides, elements
  int64_t units;                       // batch * num_query * num_heads
  int S, NH, D, NL, NQ, NP, log2_g;
};

// T: input dtype; A: arithmetic / grad_value type.
template <typename T, typename A>
__global__ void __launch_bounds__(kBlock) msda_col2im_kernel(
    const T *__restrict__ value, const T *__restrict__ loc, const T *__restrict__ attn,
    const T *__restrict__ grad_out, A *__restrict__ grad_value, T *__restrict__ grad_loc,
    T *__restrict__ grad_attn, BwdParams p) {
  const int G = 1 << p.log2_g;
  const int64_t tid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t u_raw = tid >> p.log2_g;
  // every lane of a group takes part in the butterflies: lanes of a unit past the end
  // run on the last unit with a zero gradient and store nothing
  const bool live = u_raw < p.units;
  const int64_t unit = live ? u_raw : p.units - 1;
  const int lane = (int)(tid & (G - 1));
  const int h = (int)(unit % p.NH);
  const int64_t bq = unit / p.NH;
  const int q = (int)(bq % p.NQ);
  const int b = (int)(bq / p.NQ);
  const int D = p.D, NH = p.NH;
  const int NS = p.NL * p.NP;
  const int64_t row = (int64_t)NH * D;  // elements per spatial position
  const T *go = grad_out + b * p.go_sb + q * p.go_sq + h * p.go_sh;
  // D <= G: one channel per lane, its top gradient kept in a register
  const bool one = D <= G;
  A top0 = 0;
  if (one && live && lane < D) top0 = (A)go[lane * p.go_sc];
  const T *vb = value + (int64_t)b * p.S * row + (int64_t)h * D;
  A *gvb = grad_value + (int64_t)b * p.S * row + (int64_t)h * D;
  const T *lp = loc + unit * NS * 2;
  const T *ap = attn + unit * NS;
  T *glp = grad_loc + unit * NS * 2;
  T *gap = grad_attn + unit * NS;
  for (int l = 0; l < p.NL; ++l) {
    const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
    const int64_t base = p.lsi[l];
    for (int pt = 0; pt < p.NP; ++pt) {
      const int s = l * p.NP + pt;
      const A lx = (A)lp[2 * s], ly = (A)lp[2 * s + 1], a = (A)ap[s];
      const A him = ly * (A)Hl - (A)0.5, wim = lx * (A)Wl - (A)0.5;
      A gh = 0, gw = 0, ga = 0;
      if (him > (A)-1 && wim > (A)-1 && him < (A)Hl && wim < (A)Wl) {
        const A fh = floor(him), fw = floor(wim);
        const int hl = (int)fh, wl = (int)fw;
        const A lh = him - fh, lw = wim - fw, hh = (A)1 - lh, hw = (A)1 - lw;
        const A w1 = hh * hw, w2 = hh * lw, w3 = lh * hw, w4 = lh * lw;
        const bool c1 = hl >= 0 && wl >= 0, c2 = hl >= 0 && wl + 1 <= Wl - 1;
        const bool c3 = hl + 1 <= Hl - 1 && wl >= 0;
        const bool c4 = hl + 1 <= Hl - 1 && wl + 1 <= Wl - 1;
        const int64_t o1 = (base + (int64_t)hl * Wl + wl) * row, o2 = o1 + row;
        const int64_t o3 = o1 + (int64_t)Wl * row, o4 = o3 + row;
        A sv1 = 0, sv2 = 0, sv3 = 0, sv4 = 0, sval = 0;
        for (int c = lane; c < D; c += G) {
          const A top = one ? top0 : (live ? (A)go[c * p.go_sc] : (A)0);
          const A v1 = c1 ? (A)vb[o1 + c] : (A)0, v2 = c2 ? (A)vb[o2 + c] : (A)0;
          const A v3 = c3 ? (A)vb[o3 + c] : (A)0, v4 = c4 ? (A)vb[o4 + c] : (A)0;
          const A ta = top * a;
          if (live) {
            if (c1) atomic_acc(gvb + o1 + c, w1 * ta);
            if (c2) atomic_acc(gvb + o2 + c, w2 * ta);
            if (c3) atomic_acc(gvb + o3 + c, w3 * ta);
            if (c4) atomic_acc(gvb + o4 + c, w4 * ta);
          }
          // channel sums of top*a*v per corner; the corner derivative weights are
          // uniform over the channels and applied once after the loop
          sv1 += ta * v1; sv2 += ta * v2; sv3 += ta * v3; sv4 += ta * v4;
          sval += top * (w1 * v1 + w2 * v2 + w3 * v3 + w4 * v4);
        }
        gh = (-hw * sv1 - lw * sv2 + hw * sv3 + lw * sv4) * (A)Hl;
        gw = (-hh * sv1 + hh * sv2 - lh * sv3 + lh * sv4) * (A)Wl;
        ga = sval;
      }
      for (int m = 1; m < G; m <<= 1) {
        gh += __shfl_xor(gh, m);
        gw += __shfl_xor(gw, m);
        ga += __shfl_xor(ga, m);
      }
      if (live && lane == 0) {
        glp[2 * s] = (T)gw;
        glp[2 * s + 1] = (T)gh;
        gap[s] = (T)ga;
      }
    }
  }
}

__global__ void __launch_bounds__(kBlock) fill_zero_f32(float *__restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride) p[i] = 0.f;
}

template <typename T>
__global__ void __launch_bounds__(kBlock) narrow_f32(const float *__restrict__ src,
                                                     T *__restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += stride)
    dst[i] = (T)src[i];
}

unsigned stream_grid(int64_t n) {
  const int64_t g = (n + kBlock - 1) / kBlock;
  return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

template <typename T, typename A>
hipError_t launch_t(const MsdaBwdArgs &a, A *grad_value, hipStream_t stream) {
  BwdParams p;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.units = (int64_t)a.f.batch * a.f.num_query * a.f.num_heads;
  p.S = a.f.spatial_size; p.NH = a.f.num_heads; p.D = a.f.channels;
  p.NL = a.f.num_levels; p.NQ = a.f.num_query; p.NP = a.f.num_point;
  p.log2_g = 0;
  while ((1 << p.log2_g) < a.f.channels && p.log2_g < 6) ++p.log2_g;
  const int64_t threads = p.units << p.log2_g;
  if (threads == 0) return hipSuccess;
  hipLaunchKernelGGL((msda_col2im_kernel<T, A>),
                     dim3((unsigned)((threads + kBlock - 1) / kBlock)), dim3(kBlock), 0, stream,
                     static_cast<const T *>(a.f.value), static_cast<const T *>(a.f.sampling_loc),
                     static_cast<const T *>(a.f.attn_weight),
                     static_cast<const T *>(a.grad_output), grad_value,
                     static_cast<T *>(a.grad_loc), static_cast<T *>(a.grad_attn), p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_half(const MsdaBwdArgs &a, hipStream_t stream) {
  const int64_t n = (int64_t)a.f.batch * a.f.spatial_size * a.f.num_heads * a.f.channels;
  float *acc = static_cast<float *>(a.workspace);
  hipLaunchKernelGGL(fill_zero_f32, dim3(stream_grid(n)), dim3(kBlock), 0, stream, acc, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  e = launch_t<T, float>(a, acc, stream);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((narrow_f32<T>), dim3(stream_grid(n)), dim3(kBlock), 0, stream, acc,
                     static_cast<T *>(a.grad_value), n);
  return hipGetLastError();
}

}  // namespace

int64_t msda_backward_workspace_bytes(int dtype, int64_t value_elems) {
  return (dtype == 1 || dtype == 2) ? value_elems * (int64_t)sizeof(float) : 0;
}

hipError_t launch_msda_backward(int dtype, const MsdaBwdArgs &a, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_t<float, float>(a, static_cast<float *>(a.grad_value), stream);
    case 1: return launch_half<f16>(a, stream);
    case 2: return launch_half<bf16>(a, stream);
    case 3: return launch_t<double, double>(a, static_cast<double *>(a.grad_value), stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
