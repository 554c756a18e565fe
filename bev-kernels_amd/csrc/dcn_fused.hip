// Fused NHWC DCNv2 forward for gfx950: deformable gather + GEMM with no column buffer.
// This kernel serves fp32 (v_mfma_f32_32x32x2_f32) and half types with more than 9 taps;
// fp16 / bf16 with up to 9 taps use dcn_fused_h.hip. Weights arrive in the layout of
// bevk_dcn_pack_weight: [Cout][kh][kw][C] for fp32, MFMA-fragment blocks for half types.
//
//   out[m, n] = sum_k A[m, k] * Wkc[n, k] (+ bias[n]),  m = (b, oh, ow), k = t*C + c
//   A[m, k]   = mask[m, t] * bilinear(x[b], h(m, t), w(m, t))[c]
// (naotic/bev-kernels fused_tl.py:42-139 is the algorithmic model: A tiles are built
// on the fly, never written to HBM.)
//
// Structure of one workgroup (4 waves) computing a BM x BN tile of `out`:
//   * K loop in steps of BK. Every thread owns fixed (row, 16-byte k-vector) slots of
//     the A tile; per slot it keeps the tap geometry (four corner byte offsets and
//     four mask-folded bilinear weights) and refreshes it only when the slot moves to
//     a new tap. Corner rows are read with 16-byte buffer loads; invalid corners use
//     an out-of-range offset and read zero.
//   * The blended A vectors (fp32 math, one rounding to T) and the weight tile go to
//     double-buffered LDS; one barrier per K step.
//   * The next step's global loads are issued before the current step's MFMAs
//     (v_mfma_f32_32x32x16_{f16,bf16}, or v_mfma_f32_32x32x2_f32 for fp32).
//   * Epilogue: fp32 accumulators + bias, rounded once to T.
// M tiles are dealt to XCDs in contiguous bands so that one XCD's L2 holds the rows of
// the input image its tiles sample.
#include "bevk_common.h"
#include "bevk_launch.h"

#include <hip/amd_detail/amd_hip_unsafe_atomics.h>

namespace bevk {
namespace {

constexpr int kThreads = 256;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

struct FusedParams {
  const void *x;
  const void *off;
  const void *msk;
  const void *w;
  const void *bias;
  void *out;
  const float *yb;  // kGeoYF32: fp32 bias of y (or null)
  int relu;         // max(out, 0) in the epilogue
  int B, C, H, W, Ho, Wo, Cout, kh, kw, ph, pw, sh, sw, dh, dw;
  int M, K;
  int tiles_m;
  int kz_steps;     // K steps per blockIdx.z part: two parts add into a cleared output
  uint32_t x_bytes, w_bytes;
};

// MFMA step on one 32x32 tile. A/B fragments are k-contiguous 16-byte LDS vectors.
template <typename T> struct Mfma;
template <> struct Mfma<f16> {
  static constexpr int KSTEP = 16;  // k per instruction
  __device__ static floatx16 run(const f16 *a, const f16 *b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(a),
                                                  *reinterpret_cast<const half8 *>(b), c, 0, 0, 0);
  }
};
template <> struct Mfma<bf16> {
  static constexpr int KSTEP = 16;
  __device__ static floatx16 run(const bf16 *a, const bf16 *b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8 *>(a),
                                                   *reinterpret_cast<const bf16x8 *>(b), c, 0, 0, 0);
  }
};
template <> struct Mfma<float> {
  static constexpr int KSTEP = 2;
  __device__ static floatx16 run(const float *a, const float *b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(*a, *b, c, 0, 0, 0);
  }
};
// Elements of k each lane contributes per instruction (lanes 0-31 take the first
// chunk, lanes 32-63 the second).
template <typename T> constexpr int lane_k() { return Mfma<T>::KSTEP / 2; }

// GEO: kGeoMask, kGeoY, kGeoYF32 or kGeoRegular (bevk_common.h); kGeoRegular is used
// with T = float only (the fp32 offset conv of the fused front end, fp32 bias).
template <typename T, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GEO>
__global__ void __launch_bounds__(kThreads) dcn_fused_nhwc_kernel(const FusedParams p) {
  constexpr int VEC = 16 / sizeof(T);
  constexpr int KV = BK / VEC;                    // 16-byte vectors per tile row per step
  constexpr int AV = BM * KV / kThreads;          // A vectors per thread per step
  constexpr int BV = BN * KV / kThreads;          // B vectors per thread per step
  static_assert(AV >= 1 && BV >= 1, "tile too small for the thread count");
  static_assert((BM * KV) % kThreads == 0 && (BN * KV) % kThreads == 0, "tile/thread mismatch");
  constexpr int PAD = VEC;                        // one 16-byte vector of padding per row
  constexpr int LDA = BK + PAD;
  constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(TM >= 1 && TN >= 1 && WAVES_M * WAVES_N == kThreads / kWave, "wave grid");
  using V = Vec<T, VEC>;

  __shared__ __attribute__((aligned(16))) T As[2][BM * LDA];
  __shared__ __attribute__((aligned(16))) T Bs[2][BN * LDA];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int wm = wave / WAVES_N, wn = wave - (wave / WAVES_N) * WAVES_N;

  // Contiguous band of M tiles per XCD (blocks are dealt round-robin to the 8 XCDs).
  int tile_m = blockIdx.x;
  {
    const int full = (p.tiles_m / 8) * 8;
    if (tile_m < full) tile_m = (tile_m & 7) * (full / 8) + (tile_m >> 3);
  }
  const int m0 = tile_m * BM;
  const int n0 = blockIdx.y * BN;
  // K steps [ks0, ks1) of this workgroup (the whole K unless it is split over blockIdx.z)
  const int nk = (p.K + BK - 1) / BK;
  const int ks0 = (int)blockIdx.z * p.kz_steps, ks1 = min(nk, ks0 + p.kz_steps);
  const int HoWo = p.Ho * p.Wo;
  const int T_ = p.kh * p.kw;

  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  const uint32_t xoob = p.x_bytes;
  const uint32_t woob = p.w_bytes;

  // ---- per-slot A state -------------------------------------------------------
  int a_row[AV], a_kv[AV];
  int a_m[AV];            // output pixel, or -1 past M
  int a_hb[AV], a_wb[AV]; // oh*sh - ph, ow*sw - pw
  int a_img[AV];          // b * H * W
  int a_t[AV], a_c[AV];   // current tap and channel of the slot's vector
  int a_gt[AV];           // tap of the cached geometry
  float a_w[AV][4];
  uint32_t a_o[AV][4];
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int a = tid + i * kThreads;
    a_row[i] = a / KV;
    a_kv[i] = a - (a / KV) * KV;
    const int m = m0 + a_row[i];
    a_m[i] = m < p.M ? m : -1;
    const int mm = m < p.M ? m : 0;
    const int b = mm / HoWo;
    const int r = mm - b * HoWo;
    const int oh = r / p.Wo, ow = r - (r / p.Wo) * p.Wo;
    a_hb[i] = oh * p.sh - p.ph;
    a_wb[i] = ow * p.sw - p.pw;
    a_img[i] = b * p.H * p.W;
    const int k = ks0 * BK + a_kv[i] * VEC;
    a_t[i] = k / p.C;
    a_c[i] = k - a_t[i] * p.C;
    a_gt[i] = -1;  // tap whose geometry is cached: none yet
  }

  auto refresh_geometry = [&](int i, int t) {
    const int m = a_m[i];
    float w1 = 0.f, w2 = 0.f, w3 = 0.f, w4 = 0.f;
    uint32_t o1 = xoob, o2 = xoob, o3 = xoob, o4 = xoob;
    if (GEO == kGeoRegular && m >= 0 && t < T_) {
      const int ki = t / p.kw, kj = t - (t / p.kw) * p.kw;
      const int h = a_hb[i] + ki * p.dh, w = a_wb[i] + kj * p.dw;
      if (h >= 0 && h < p.H && w >= 0 && w < p.W) {
        w1 = 1.f;
        o1 = (uint32_t)(a_img[i] + h * p.W + w) * (uint32_t)p.C * (uint32_t)sizeof(T);
      }
    } else if (m >= 0 && t < T_) {
      float dy, dx, mk;
      tap_offsets<T, GEO>(p.off, p.msk, p.yb, m, t, T_, dy, dx, mk);
      const int ki = t / p.kw, kj = t - (t / p.kw) * p.kw;
      const float h = (float)(a_hb[i] + ki * p.dh) + dy;
      const float w = (float)(a_wb[i] + kj * p.dw) + dx;
      if (h > -1.f && w > -1.f && h < (float)p.H && w < (float)p.W) {
        const float fh = floorf(h), fw = floorf(w);
        const int hl = (int)fh, wl = (int)fw;
        const float lh = h - fh, lw = w - fw, hh = 1.f - lh, hw = 1.f - lw;
        const bool y0 = hl >= 0, y1 = hl + 1 <= p.H - 1;
        const bool x0 = wl >= 0, x1 = wl + 1 <= p.W - 1;
        const uint32_t row = (uint32_t)p.C * (uint32_t)sizeof(T);
        const uint32_t base = (uint32_t)(a_img[i] + hl * p.W + wl) * row;
        if (y0 && x0) { w1 = hh * hw * mk; o1 = base; }
        if (y0 && x1) { w2 = hh * lw * mk; o2 = base + row; }
        if (y1 && x0) { w3 = lh * hw * mk; o3 = base + (uint32_t)p.W * row; }
        if (y1 && x1) { w4 = lh * lw * mk; o4 = base + (uint32_t)(p.W + 1) * row; }
      }
    }
    a_w[i][0] = w1; a_w[i][1] = w2; a_w[i][2] = w3; a_w[i][3] = w4;
    a_o[i][0] = o1; a_o[i][1] = o2; a_o[i][2] = o3; a_o[i][3] = o4;
  };

  // Raw global data for one K step, held in registers between issue and use.
  V ra[AV][4];
  V rb[BV];

  auto issue_loads = [&](int ks) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      // Advance the slot's (t, c) to k = ks*BK + kv*VEC.
      if (ks > ks0) {
        a_c[i] += BK;
        while (a_c[i] >= p.C) { a_c[i] -= p.C; ++a_t[i]; }
      }
      if (a_t[i] != a_gt[i]) {
        refresh_geometry(i, a_t[i]);
        a_gt[i] = a_t[i];
      }
      const uint32_t cb = (uint32_t)a_c[i] * (uint32_t)sizeof(T);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t o = a_o[i][q];
        ra[i][q] = buffer_load_vec<T, VEC>(xr, o == xoob ? xoob : o + cb);
      }
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int v = tid + i * kThreads;
      const int n = n0 + v / KV;
      const int k = ks * BK + (v - (v / KV) * KV) * VEC;
      const bool ok = n < p.Cout && k < p.K;
      uint32_t o = woob;
      if (ok) {
        if constexpr (sizeof(T) == 4) {
          o = ((uint32_t)n * (uint32_t)p.K + (uint32_t)k) * 4u;  // [Cout][K]
        } else {
          // fragment-packed: block (n/32, k/16), lane (n%32) + 32 * ((k%16)/8), 16 B each
          const uint32_t kb_total = (uint32_t)(p.K + 15) / 16u;
          o = (((uint32_t)(n >> 5) * kb_total + (uint32_t)(k >> 4)) * 64u + (uint32_t)(n & 31) +
               32u * (uint32_t)((k & 15) >> 3)) * 16u;
        }
      }
      rb[i] = buffer_load_vec<T, VEC>(wr, o);
    }
  };

  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      V o;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const float val = a_w[i][0] * (float)ra[i][0].v[e] + a_w[i][1] * (float)ra[i][1].v[e] +
                          a_w[i][2] * (float)ra[i][2].v[e] + a_w[i][3] * (float)ra[i][3].v[e];
        o.v[e] = static_cast<T>(val);
      }
      store_vec<T, VEC>(&As[buf][a_row[i] * LDA + a_kv[i] * VEC], o);
    }
#pragma unroll
    for (int i = 0; i < BV; ++i) {
      const int v = tid + i * kThreads;
      store_vec<T, VEC>(&Bs[buf][(v / KV) * LDA + (v - (v / KV) * KV) * VEC], rb[i]);
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int lrow = lane & 31;
  const int lk = (lane >> 5) * lane_k<T>();

  issue_loads(ks0);
  for (int ks = ks0; ks < ks1; ++ks) {
    const int buf = (ks - ks0) & 1;
    store_lds(buf);
    __syncthreads();
    if (ks + 1 < ks1) issue_loads(ks + 1);
#pragma unroll
    for (int kk = 0; kk < BK; kk += Mfma<T>::KSTEP) {
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const T *a = &As[buf][(wm * WTM + i * 32 + lrow) * LDA + kk + lk];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const T *bp = &Bs[buf][(wn * WTN + j * 32 + lrow) * LDA + kk + lk];
          acc[i][j] = Mfma<T>::run(a, bp, acc[i][j]);
        }
      }
    }
  }

  // ---- epilogue: D[row][col], lane holds col = lane%32,
  //      row = 8*(e/4) + 4*(lane/32) + e%4 for e in [0, 16).
  //      Split K (fp32 only, no ReLU): each part adds its sum to the cleared output, the
  //      bias with the first part; with two parts the result does not depend on their
  //      order (0 + a + b == 0 + b + a).
  T *out = static_cast<T *>(p.out);
  const T *bias = static_cast<const T *>(p.bias);
  const bool split = gridDim.z > 1;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + wn * WTN + j * 32 + lrow;
    const float bv = (bias != nullptr && n < p.Cout && blockIdx.z == 0) ? (float)bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int row = wm * WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int m = m0 + row;
        float v = acc[i][j][e] + bv;
        if (GEO != kGeoRegular && p.relu) v = v < 0.f ? 0.f : v;  // NaN stays NaN
        if (m < p.M && n < p.Cout) {
          if (sizeof(T) == 4 && split)
            unsafeAtomicAdd(reinterpret_cast<float *>(out) + (int64_t)m * p.Cout + n, v);
          else
            out[(int64_t)m * p.Cout + n] = static_cast<T>(v);
        }
      }
    }
  }
}

template <typename T, int BM, int BN, int BK, int WM, int WN>
hipError_t launch_cfg(const FusedParams &p, int geo, hipStream_t stream) {
  const int nk = (p.K + BK - 1) / BK;
  dim3 grid(p.tiles_m, (p.Cout + BN - 1) / BN, (nk + p.kz_steps - 1) / p.kz_steps);
  if (geo == kGeoY)
    hipLaunchKernelGGL((dcn_fused_nhwc_kernel<T, BM, BN, BK, WM, WN, kGeoY>), grid,
                       dim3(kThreads), 0, stream, p);
  else if (geo == kGeoYF32)
    hipLaunchKernelGGL((dcn_fused_nhwc_kernel<T, BM, BN, BK, WM, WN, kGeoYF32>), grid,
                       dim3(kThreads), 0, stream, p);
  else if (geo == kGeoRegular && sizeof(T) == 4)
    hipLaunchKernelGGL((dcn_fused_nhwc_kernel<T, BM, BN, BK, WM, WN, kGeoRegular>), grid,
                       dim3(kThreads), 0, stream, p);
  else if (geo == kGeoMask)
    hipLaunchKernelGGL((dcn_fused_nhwc_kernel<T, BM, BN, BK, WM, WN, kGeoMask>), grid,
                       dim3(kThreads), 0, stream, p);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

__global__ void __launch_bounds__(kThreads) fill_zero_f32x4(float *__restrict__ p, int64_t n4) {
  for (int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x; i < n4;
       i += (int64_t)gridDim.x * kThreads)
    reinterpret_cast<float4 *>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
}

template <typename T>
hipError_t launch_t(FusedParams p, int geo, hipStream_t stream) {
  constexpr int BK = sizeof(T) == 4 ? 16 : 32;
  constexpr int BM = 64;
  p.tiles_m = (p.M + BM - 1) / BM;
  const int nk = (p.K + BK - 1) / BK;
  p.kz_steps = nk;
  // fp32 with fewer than three workgroups per CU (res4: 544 tiles, res5: 272) and no ReLU:
  // K in two halves that add into the cleared output, twice the workgroups (res4 fp32
  // 505 -> 465 us, res5 665 -> 517 us)
  const int bn = p.Cout > 128 ? 256 : p.Cout > 64 ? 128 : 64;  // BN of the launch below
  const int64_t tiles = (int64_t)p.tiles_m * ((p.Cout + bn - 1) / bn);
  const int64_t n_out = (int64_t)p.M * p.Cout;
  if (sizeof(T) == 4 && !p.relu && nk >= 64 && tiles < 3 * (int64_t)device_cus() &&
      n_out % 4 == 0 && reinterpret_cast<uintptr_t>(p.out) % 16 == 0) {
    p.kz_steps = (nk + 1) / 2;
    const int64_t n4 = n_out / 4;
    const unsigned g = (unsigned)std::min<int64_t>((n4 + kThreads - 1) / kThreads, 8192);
    hipLaunchKernelGGL(fill_zero_f32x4, dim3(g), dim3(kThreads), 0, stream,
                       static_cast<float *>(p.out), n4);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.Cout > 128) return launch_cfg<T, BM, 256, BK, 1, 4>(p, geo, stream);
  if (p.Cout > 64) return launch_cfg<T, BM, 128, BK, 1, 4>(p, geo, stream);
  return launch_cfg<T, BM, 64, BK, 2, 2>(p, geo, stream);
}

}  // namespace

hipError_t launch_dcn_fused_nhwc(int dtype, const DcnGeom &g, int channels_out, const void *x,
                                 const void *off, int geo, const void *msk,
                                 const void *w_packed, const void *bias, void *out,
                                 hipStream_t stream, const float *y_bias, bool relu) {
  if (dtype != 0 && dcn_fused_h_supported(g))
    return launch_dcn_fused_h(dtype, g, channels_out, x, off, geo, msk, w_packed, bias, out,
                              stream, y_bias, relu);
  if (dtype != 0 && geo == kGeoRegular) return hipErrorInvalidValue;  // fp32 output only
  FusedParams p;
  p.x = x; p.off = off; p.msk = msk; p.w = w_packed; p.bias = bias; p.out = out;
  p.yb = y_bias; p.relu = relu ? 1 : 0;
  p.B = g.batch; p.C = g.channels; p.H = g.height; p.W = g.width;
  p.Ho = g.height_col; p.Wo = g.width_col; p.Cout = channels_out;
  p.kh = g.kernel_h; p.kw = g.kernel_w; p.ph = g.pad_h; p.pw = g.pad_w;
  p.sh = g.stride_h; p.sw = g.stride_w; p.dh = g.dil_h; p.dw = g.dil_w;
  p.M = g.batch * g.height_col * g.width_col;
  p.K = g.kernel_h * g.kernel_w * g.channels;
  p.tiles_m = 0;
  const int es = dtype == 0 ? 4 : 2;
  p.x_bytes = (uint32_t)((int64_t)g.batch * g.height * g.width * g.channels * es);
  p.w_bytes = (uint32_t)(dtype == 0 ? (int64_t)channels_out * p.K * 4
                                    : dcn_packed_weight_elems(dtype, channels_out, p.K) * 2);
  switch (dtype) {
    case 0: return launch_t<float>(p, geo, stream);
    case 1: return launch_t<f16>(p, geo, stream);
    case 2: return launch_t<bf16>(p, geo, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
