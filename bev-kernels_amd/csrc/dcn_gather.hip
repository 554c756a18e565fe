// DCNv2 modulated deformable gathers ("im2col") for gfx950, NCHW and NHWC.
//
// Semantics (naotic/bev-kernels modulated_deform_conv.py:184-266, fused_tl.py:146-201):
//   h = oh*s_h - p_h + i*d_h + off[2t],  w = ow*s_w - p_w + j*d_w + off[2t+1],  t = i*kw + j
//   the tap is zero unless -1 < h < H and -1 < w < W; otherwise it is the bilinear blend
//   of the four neighbours, each neighbour zero outside [0,H-1] x [0,W-1], times mask[t].
//
// Both kernels read the input through a raw buffer descriptor per image: an invalid
// neighbour gets an out-of-range offset, which returns 0 without touching memory, so
// the zero padding costs no branch and no wasted load.
#include "bevk_common.h"
#include "bevk_launch.h"

namespace bevk {
namespace {

constexpr int kBlock = 256;

// Bilinear tap geometry shared by the gathers. Offsets are element indices within
// one image plane (NCHW) or one image (NHWC, multiplied by channels by the caller).
template <typename A>
struct Tap {
  A w1, w2, w3, w4;      // corner weights, zero for invalid corners
  int i1, i2, i3, i4;    // corner positions y*W + x, or -1 when invalid
};

template <typename A>
__device__ __forceinline__ Tap<A> make_tap(A h, A w, int H, int W) {
  Tap<A> tp;
  tp.w1 = tp.w2 = tp.w3 = tp.w4 = (A)0;
  tp.i1 = tp.i2 = tp.i3 = tp.i4 = -1;
  if (h > (A)-1 && w > (A)-1 && h < (A)H && w < (A)W) {
    const A fh = floor(h), fw = floor(w);
    const int hl = (int)fh, wl = (int)fw;
    const A lh = h - fh, lw = w - fw;
    const A hh = (A)1 - lh, hw = (A)1 - lw;
    const bool y0 = hl >= 0, y1 = hl + 1 <= H - 1;
    const bool x0 = wl >= 0, x1 = wl + 1 <= W - 1;
    const int p = hl * W + wl;
    if (y0 && x0) { tp.w1 = hh * hw; tp.i1 = p; }
    if (y0 && x1) { tp.w2 = hh * lw; tp.i2 = p + 1; }
    if (y1 && x0) { tp.w3 = lh * hw; tp.i3 = p + W; }
    if (y1 && x1) { tp.w4 = lh * lw; tp.i4 = p + W + 1; }
  }
  return tp;
}

// ---------------------------------------------------------------------------
// NCHW: col[(c*T + t), b, oh, ow]. One thread per (b, spatial position, tap) and a
// run of `cpc` channels of one deformable group: the geometry is computed once and
// reused over the channel run; consecutive threads are consecutive output columns,
// so the column writes and the offset / mask reads are coalesced.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kBlock) im2col_nchw_kernel(
    const T *__restrict__ im, const T *__restrict__ offset, const T *__restrict__ mask,
    T *__restrict__ col, const DcnGeom g, int chunks_per_group, int cpc, uint32_t img_bytes) {
  using A = typename Acc<T>::type;
  const int HoWo = g.height_col * g.width_col;
  const int sp = blockIdx.x * kBlock + threadIdx.x;
  if (sp >= HoWo) return;
  const int b = blockIdx.y;
  const int T_ = g.kernel_h * g.kernel_w;
  int z = blockIdx.z;
  const int t = z % T_;
  z /= T_;
  const int chunk = z % chunks_per_group;
  const int dgi = z / chunks_per_group;
  const int cpg = g.channels / g.deformable_group;
  const int c_begin = dgi * cpg + chunk * cpc;
  const int c_end = min(c_begin + cpc, (dgi + 1) * cpg);
  const int oh = sp / g.width_col, ow = sp - oh * g.width_col;
  const int i = t / g.kernel_w, j = t - i * g.kernel_w;

  const int64_t om_base = (int64_t)b * g.deformable_group + dgi;
  const A dy = (A)offset[(om_base * 2 * T_ + 2 * t) * HoWo + sp];
  const A dx = (A)offset[(om_base * 2 * T_ + 2 * t + 1) * HoWo + sp];
  const A mk = (A)mask[(om_base * T_ + t) * HoWo + sp];
  const A h = (A)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
  const A w = (A)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
  const Tap<A> tp = make_tap<A>(h, w, g.height, g.width);

  const __amdgpu_buffer_rsrc_t rsrc =
      make_rsrc(im + (int64_t)b * g.channels * g.height * g.width, img_bytes);
  const uint32_t plane = (uint32_t)(g.height * g.width);
  const uint32_t oob = img_bytes;
  auto boff = [&](int idx, int c) -> uint32_t {
    return idx < 0 ? oob : ((uint32_t)c * plane + (uint32_t)idx) * (uint32_t)sizeof(T);
  };
  const int64_t row_stride = (int64_t)g.batch * HoWo;
  T *out = col + ((int64_t)c_begin * T_ + t) * row_stride + (int64_t)b * HoWo + sp;
  for (int c = c_begin; c < c_end; ++c) {
    const A v1 = (A)buffer_load_one<T>(rsrc, boff(tp.i1, c));
    const A v2 = (A)buffer_load_one<T>(rsrc, boff(tp.i2, c));
    const A v3 = (A)buffer_load_one<T>(rsrc, boff(tp.i3, c));
    const A v4 = (A)buffer_load_one<T>(rsrc, boff(tp.i4, c));
    const A val = tp.w1 * v1 + tp.w2 * v2 + tp.w3 * v3 + tp.w4 * v4;
    *out = static_cast<T>(val * mk);
    out += T_ * row_stride;
  }
}

// ---------------------------------------------------------------------------
// NHWC (dg == 1): col[m, t*C + c], m = (b, oh, ow). A wave owns kPPW consecutive (m, t)
// pairs of one image. Lane i < kPPW first computes the geometry of pair i (offsets and
// mask read once, bilinear weights, corner byte offsets) into LDS; then groups of LPP
// lanes take the wave's pairs in turn and sweep the channels with 16-byte loads of the
// four corner rows, so each pair costs four gathers and one store per channel chunk and
// no per-lane geometry loads; kPPW = 16 keeps enough waves and loads in flight. Consecutive pairs are consecutive taps of one pixel, so one
// pixel's 9*C column row is written contiguously.
// ---------------------------------------------------------------------------
constexpr int kPPW = 16;  // pairs per wave

struct PairGeo {
  float w[4];   // corner weights (zero for invalid corners)
  float mk;     // mask (applied after the blend, as the column is defined)
  uint32_t o[4];  // corner byte offsets in the image, out of range when invalid
};

template <typename T, int VEC, bool FUSED_Y, typename Y>
__global__ void __launch_bounds__(kBlock) im2col_nhwc_kernel(
    const T *__restrict__ im, const Y *__restrict__ offset, const T *__restrict__ mask,
    T *__restrict__ col, const DcnGeom g, int lpp_log2, uint32_t img_bytes,
    const float *__restrict__ y_bias, int chunks) {
  __shared__ PairGeo geo[kBlock / kWave * kPPW];
  const int T_ = g.kernel_h * g.kernel_w;
  const int HoWo = g.height_col * g.width_col;
  // Block l runs on XCD l % 8 and takes chunk (l % 8) * (n / 8) + l / 8 of the n =
  // batch * chunks chunks (n a multiple of 8), so each XCD gathers from one contiguous
  // range of pixels and the input rows stay in its L2.
  const int n8 = (int)(gridDim.x >> 3);
  const int cid = (int)(blockIdx.x & 7) * n8 + (int)(blockIdx.x >> 3);
  const int b = cid / chunks;
  if (b >= g.batch) return;  // padding chunks
  const int chunk = cid - b * chunks;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int npairs = HoWo * T_;
  const int pbase = (chunk * (kBlock / kWave) + wave) * kPPW;  // first pair of the wave
  if (pbase >= npairs) return;                           // uniform over the wave
  const int C = g.channels;
  const uint32_t oob = img_bytes;
  const uint32_t row = (uint32_t)C * (uint32_t)sizeof(T);

  // Phase 1: geometry of pair pbase + lane.
  if (lane < kPPW) {
    const int pair = pbase + lane;
    PairGeo G;
    G.w[0] = G.w[1] = G.w[2] = G.w[3] = 0.f;
    G.mk = 0.f;
    G.o[0] = G.o[1] = G.o[2] = G.o[3] = oob;
    if (pair < npairs) {
      const int sp = pair / T_, t = pair - (pair / T_) * T_;
      const int oh = sp / g.width_col, ow = sp - oh * g.width_col;
      const int i = t / g.kernel_w, j = t - i * g.kernel_w;
      const int64_t m = (int64_t)b * HoWo + sp;
      float dy, dx, mk;
      if constexpr (FUSED_Y) {  // y [B, Ho, Wo, 3T]: offsets then pre-sigmoid mask
        const Y *yp = offset + m * 3 * T_;
        dy = (float)yp[2 * t];
        dx = (float)yp[2 * t + 1];
        float ym = (float)yp[2 * T_ + t];
        if (y_bias != nullptr) {
          dy += y_bias[2 * t];
          dx += y_bias[2 * t + 1];
          ym += y_bias[2 * T_ + t];
        }
        mk = sigmoid_f32(ym);
      } else {
        dy = (float)offset[m * 2 * T_ + 2 * t];
        dx = (float)offset[m * 2 * T_ + 2 * t + 1];
        mk = (float)mask[m * T_ + t];
      }
      const float h = (float)(oh * g.stride_h - g.pad_h + i * g.dil_h) + dy;
      const float w = (float)(ow * g.stride_w - g.pad_w + j * g.dil_w) + dx;
      const Tap<float> tp = make_tap<float>(h, w, g.height, g.width);
      G.w[0] = tp.w1; G.w[1] = tp.w2; G.w[2] = tp.w3; G.w[3] = tp.w4;
      G.mk = mk;
      G.o[0] = tp.i1 < 0 ? oob : (uint32_t)tp.i1 * row;
      G.o[1] = tp.i2 < 0 ? oob : (uint32_t)tp.i2 * row;
      G.o[2] = tp.i3 < 0 ? oob : (uint32_t)tp.i3 * row;
      G.o[3] = tp.i4 < 0 ? oob : (uint32_t)tp.i4 * row;
    }
    geo[wave * kPPW + lane] = G;
  }
  // The wave reads what its own lanes wrote: order the LDS accesses within the wave.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // Phase 2: lane group gi (LPP lanes) takes pairs gi, gi + PPI, ... of the wave. An
  // out-of-range corner offset stays out of range with the channel offset added
  // (img_bytes < 2^31), so every load is issued unconditionally.
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(im + (int64_t)b * g.height * g.width * C, img_bytes);
  const int LPP = 1 << lpp_log2;
  const int PPI = kWave >> lpp_log2;  // pairs per iteration
  const int li = lane & (LPP - 1), gi = lane >> lpp_log2;
  const int nk = min(kPPW, npairs - pbase);
  using V = Vec<T, VEC>;
#pragma unroll 4
  for (int k = gi; k < nk; k += PPI) {
    const PairGeo G = geo[wave * kPPW + k];
    const int pair = pbase + k;
    const int sp = pair / T_, t = pair - (pair / T_) * T_;
    T *out = col + ((int64_t)b * HoWo + sp) * T_ * C + (int64_t)t * C;
    for (int c = li * VEC; c < C; c += LPP * VEC) {
      const uint32_t cb = (uint32_t)c * (uint32_t)sizeof(T);
      V v1, v2, v3, v4;
      if constexpr (VEC > 1) {
        v1 = buffer_load_vec<T, VEC>(rsrc, G.o[0] + cb);
        v2 = buffer_load_vec<T, VEC>(rsrc, G.o[1] + cb);
        v3 = buffer_load_vec<T, VEC>(rsrc, G.o[2] + cb);
        v4 = buffer_load_vec<T, VEC>(rsrc, G.o[3] + cb);
      } else {
        v1.v[0] = buffer_load_one<T>(rsrc, G.o[0] + cb);
        v2.v[0] = buffer_load_one<T>(rsrc, G.o[1] + cb);
        v3.v[0] = buffer_load_one<T>(rsrc, G.o[2] + cb);
        v4.v[0] = buffer_load_one<T>(rsrc, G.o[3] + cb);
      }
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float val = G.w[0] * (float)v1.v[e] + G.w[1] * (float)v2.v[e] +
                          G.w[2] * (float)v3.v[e] + G.w[3] * (float)v4.v[e];
        o.v[e] = static_cast<T>(val * G.mk);
      }
      store_vec<T, VEC>(out + c, o);
    }
  }
}

template <typename T>
hipError_t launch_nchw_t(const DcnGeom &g, const void *im, const void *off, const void *msk,
                         void *col, bool tiled, hipStream_t stream) {
  const int HoWo = g.height_col * g.width_col;
  const int T_ = g.kernel_h * g.kernel_w;
  const int cpg = g.channels / g.deformable_group;
  // Channels per thread: 1 for the per-channel kernel; the tiled kernel reuses the
  // geometry over up to 16 channels while keeping >= ~8 waves per CU in flight.
  int cpc = 1;
  if (tiled) {
    cpc = 16;
    while (cpc > 1 && (int64_t)g.batch * HoWo * T_ * ((cpg + cpc - 1) / cpc) < 256LL * 8 * 64)
      cpc /= 2;
  }
  int chunks = (cpg + cpc - 1) / cpc;
  while ((int64_t)g.deformable_group * chunks * T_ > 65535) {  // grid.z limit
    cpc *= 2;
    chunks = (cpg + cpc - 1) / cpc;
  }
  const uint32_t img_bytes = (uint32_t)((int64_t)g.channels * g.height * g.width * sizeof(T));
  dim3 grid((HoWo + kBlock - 1) / kBlock, g.batch, g.deformable_group * chunks * T_);
  hipLaunchKernelGGL(im2col_nchw_kernel<T>, grid, dim3(kBlock), 0, stream,
                     static_cast<const T *>(im), static_cast<const T *>(off),
                     static_cast<const T *>(msk), static_cast<T *>(col), g, chunks, cpc,
                     img_bytes);
  return hipGetLastError();
}

template <typename T, bool FY, typename Y = T>
hipError_t launch_nhwc_t(const DcnGeom &g, const void *im, const void *off, const void *msk,
                         void *col, hipStream_t stream, const float *y_bias = nullptr) {
  constexpr int VEC = 16 / sizeof(T);
  const int C = g.channels;
  const bool vec = (C % VEC) == 0;
  const int per_lane = vec ? VEC : 1;
  int lpp = 1;
  while (lpp < 64 && lpp * per_lane < C) lpp *= 2;
  int lpp_log2 = 0;
  while ((1 << lpp_log2) < lpp) ++lpp_log2;
  const int T_ = g.kernel_h * g.kernel_w;
  const int64_t pairs = (int64_t)g.height_col * g.width_col * T_;
  constexpr int kPairsPerBlock = kBlock / kWave * kPPW;
  const int chunks = (int)((pairs + kPairsPerBlock - 1) / kPairsPerBlock);
  const int64_t nblk = ((int64_t)chunks * g.batch + 7) / 8 * 8;
  dim3 grid((unsigned)nblk);
  const uint32_t img_bytes = (uint32_t)((int64_t)g.height * g.width * C * sizeof(T));
  if (vec)
    hipLaunchKernelGGL((im2col_nhwc_kernel<T, VEC, FY, Y>), grid, dim3(kBlock), 0, stream,
                       static_cast<const T *>(im), static_cast<const Y *>(off),
                       static_cast<const T *>(msk), static_cast<T *>(col), g, lpp_log2,
                       img_bytes, y_bias, chunks);
  else
    hipLaunchKernelGGL((im2col_nhwc_kernel<T, 1, FY, Y>), grid, dim3(kBlock), 0, stream,
                       static_cast<const T *>(im), static_cast<const Y *>(off),
                       static_cast<const T *>(msk), static_cast<T *>(col), g, lpp_log2,
                       img_bytes, y_bias, chunks);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_im2col_nchw(int dtype, const DcnGeom &g, const void *im, const void *off,
                              const void *msk, void *col, bool tiled, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_nchw_t<float>(g, im, off, msk, col, tiled, stream);
    case 1: return launch_nchw_t<f16>(g, im, off, msk, col, tiled, stream);
    case 2: return launch_nchw_t<bf16>(g, im, off, msk, col, tiled, stream);
    case 3: return launch_nchw_t<double>(g, im, off, msk, col, tiled, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_im2col_nhwc(int dtype, const DcnGeom &g, const void *im, const void *off,
                              bool fused_y, const void *msk, void *col, hipStream_t stream) {
  switch (dtype) {
    case 0: return fused_y ? launch_nhwc_t<float, true>(g, im, off, msk, col, stream)
                           : launch_nhwc_t<float, false>(g, im, off, msk, col, stream);
    case 1: return fused_y ? launch_nhwc_t<f16, true>(g, im, off, msk, col, stream)
                           : launch_nhwc_t<f16, false>(g, im, off, msk, col, stream);
    case 2: return fused_y ? launch_nhwc_t<bf16, true>(g, im, off, msk, col, stream)
                           : launch_nhwc_t<bf16, false>(g, im, off, msk, col, stream);
    case 3: return fused_y ? launch_nhwc_t<double, true>(g, im, off, msk, col, stream)
                           : launch_nhwc_t<double, false>(g, im, off, msk, col, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_im2col_nhwc_yf32(int dtype, const DcnGeom &g, const void *im, const float *y,
                                   const float *y_bias, void *col, hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_nhwc_t<float, true, float>(g, im, y, nullptr, col, stream, y_bias);
    case 1: return launch_nhwc_t<f16, true, float>(g, im, y, nullptr, col, stream, y_bias);
    case 2: return launch_nhwc_t<bf16, true, float>(g, im, y, nullptr, col, stream, y_bias);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
