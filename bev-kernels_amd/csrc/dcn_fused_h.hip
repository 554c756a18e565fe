// Fused NHWC DCNv2 forward for fp16 / bf16 on gfx950 (kernels with at most 9 taps).
//
//   out[m, n] = sum_k A[m, k] * W[n, k] (+ bias[n]),  m = (b, oh, ow), k = t*C + c
//   A[m, k]   = mask[m, t] * bilinear(x[b], h(m, t), w(m, t))[c]
//
// Structure of one workgroup (4 waves, BM x BN output tile):
//   * Geometry table: at start, each (tile row, tap) pair gets its four corner byte
//     offsets (out-of-range sentinel if the corner is outside the image) and four
//     bilinear x mask weights, once, in LDS.
//   * A operand: per K step (BK = 64 channels of one tap) each thread gathers 16-byte
//     vectors of the four corner rows of its (row, k-vector) slots with buffer loads
//     (8 lanes cover 128 contiguous bytes of a pixel), blends them in fp32 with one
//     rounding to T (blend4) and writes the A tile to double-buffered LDS.
//   * B operand: the weight is pre-packed in MFMA fragment order, so every B fragment is
//     one coalesced 1 KB load straight into registers (double-buffered across K steps).
//     LDS only carries the A tile.
//   * MFMA v_mfma_f32_32x32x16_{f16,bf16}: each wave owns a 64 x 64 block of the tile.
//   * Epilogue: fp32 accumulators + bias, one rounding to T.
//   * Tile order: block b runs on XCD b % 8; each XCD takes a contiguous range of output
//     tiles, so the image rows its tiles gather from stay in that XCD's L2.
#include "bevk_common.h"
#include "bevk_launch.h"

#include <hip/amd_detail/amd_hip_unsafe_atomics.h>

#include <algorithm>
#include <type_traits>

namespace bevk {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int int4v __attribute__((ext_vector_type(4)));

constexpr int kMaxTaps = 9;

struct HParams {
  const void *x, *off, *msk, *w, *bias;
  void *out;
  const float *yb;               // kGeoYF32: fp32 bias of y (or null)
  int relu;                      // max(out, 0) in the epilogue
  int C, H, W, Ho, Wo, Cout, kh, kw, ph, pw, sh, sw, dh, dw, M, K;
  int taps, nb_total, kb_total;  // packed weight blocks: [nb_total][kb_total][64][16 B]
  int mt, nt, tiles_per_xcd;     // output tiles (M x N) and tiles per XCD
  int kz_steps;                  // K steps per blockIdx.y part (fp32 output: two parts add
                                 // into the cleared output; else the whole K)
  uint32_t x_bytes, w_bytes;
  // offset conv of the one-launch forward: packed w_off (3T <= 32 columns, one 32-column
  // fragment block), its fp32 bias and the fp32 y [M][3T] written out (or null)
  const void *w2;
  const float *b2;
  float *y_out;
  uint32_t w2_bytes;
};

template <typename T> __device__ __forceinline__ floatx16 mfma16(const T *a, int4v b, floatx16 c);
template <> __device__ __forceinline__ floatx16 mfma16<f16>(const f16 *a, int4v b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8 *>(a),
                                                __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ floatx16 mfma16<bf16>(const bf16 *a, int4v b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8 *>(a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// The same MFMA with the A fragment already in registers.
template <typename T> __device__ __forceinline__ floatx16 mfma16r(int4v a, int4v b, floatx16 c) {
  if constexpr (std::is_same<T, f16>::value)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a),
                                                  __builtin_bit_cast(half8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

struct TapGeo {
  float w[4];
  uint32_t o[4];
};

// A tap that contributes nothing: zero weights, every corner out of range.
__device__ __forceinline__ TapGeo empty_geo(uint32_t oob) {
  TapGeo G;
  G.w[0] = G.w[1] = G.w[2] = G.w[3] = 0.f;
  G.o[0] = G.o[1] = G.o[2] = G.o[3] = oob;
  return G;
}

// Deformable sample at (h, w) of image b: corner byte offsets (row = C elements of T) and
// mask-folded bilinear weights. The whole sample is zero unless -1 < h < H and -1 < w < W
// (modulated_deform_conv.py:256-258); each corner outside the image is zero
// (fused_tl.py:146-174, dcn_fused_nhwc_kernel.cuh:140-187).
template <typename T>
__device__ __forceinline__ TapGeo deform_geo(float h, float w, float mk, int b, int H, int W,
                                             int C, uint32_t oob) {
  TapGeo G = empty_geo(oob);
  if (h > -1.f && w > -1.f && h < (float)H && w < (float)W) {
    const float fh = floorf(h), fw = floorf(w);
    const int hl = (int)fh, wl = (int)fw;
    const float lh = h - fh, lw = w - fw, hh = 1.f - lh, hw = 1.f - lw;
    const uint32_t rowb = (uint32_t)C * (uint32_t)sizeof(T);
    const uint32_t base = (uint32_t)(b * H * W + hl * W + wl) * rowb;
    const bool y0 = hl >= 0, y1 = hl + 1 <= H - 1, x0 = wl >= 0, x1 = wl + 1 <= W - 1;
    if (y0 && x0) { G.w[0] = hh * hw * mk; G.o[0] = base; }
    if (y0 && x1) { G.w[1] = hh * lw * mk; G.o[1] = base + rowb; }
    if (y1 && x0) { G.w[2] = lh * hw * mk; G.o[2] = base + (uint32_t)W * rowb; }
    if (y1 && x1) { G.w[3] = lh * lw * mk; G.o[3] = base + (uint32_t)(W + 1) * rowb; }
  }
  return G;
}

// Plain convolution tap (the offset conv): the one in-image pixel with weight 1.
template <typename T>
__device__ __forceinline__ TapGeo regular_geo(int h, int w, int b, int H, int W, int C,
                                              uint32_t oob) {
  TapGeo G = empty_geo(oob);
  if (h >= 0 && h < H && w >= 0 && w < W) {
    G.w[0] = 1.f;
    G.o[0] = (uint32_t)(b * H * W + h * W + w) * (uint32_t)C * (uint32_t)sizeof(T);
  }
  return G;
}

// Geometry of tap t of output row m (m < M) in form GEO; for the y forms `off` is y.
template <typename T, int GEO>
__device__ __forceinline__ TapGeo tap_geo(const HParams &p, const void *off, int64_t ym, int m,
                                          int t) {
  const int HoWo = p.Ho * p.Wo;
  const int b = m / HoWo, r = m - b * HoWo, oh = r / p.Wo, ow = r - (r / p.Wo) * p.Wo;
  const int ki = t / p.kw, kj = t - (t / p.kw) * p.kw;
  const int h0 = oh * p.sh - p.ph + ki * p.dh, w0 = ow * p.sw - p.pw + kj * p.dw;
  if constexpr (GEO == kGeoRegular) {
    return regular_geo<T>(h0, w0, b, p.H, p.W, p.C, p.x_bytes);
  } else {
    float dy, dx, mk;
    tap_offsets<T, GEO>(off, p.msk, p.yb, ym, t, p.taps, dy, dx, mk);
    return deform_geo<T>((float)h0 + dy, (float)w0 + dx, mk, b, p.H, p.W, p.C, p.x_bytes);
  }
}

// One A-tile vector: sum_q w_q * corner_q in fp32 (the corners converted exactly), rounded
// once to T, as the reference's gather does (dcn_fused_nhwc_kernel.cuh:185-187,
// fused_tl.py:128-133). For fp16 the compiler takes the corners straight from their
// halves (v_fma_mix_f32); the fma with a zero addend keeps the first product in that form.
template <typename T>
__device__ __forceinline__ Vec<T, 8> blend4(const Vec<T, 8> (&c)[4], float w0, float w1,
                                            float w2, float w3) {
  Vec<T, 8> o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float s = __builtin_fmaf(w0, (float)c[0].v[e], 0.f);
    s = __builtin_fmaf(w1, (float)c[1].v[e], s);
    s = __builtin_fmaf(w2, (float)c[2].v[e], s);
    s = __builtin_fmaf(w3, (float)c[3].v[e], s);
    o.v[e] = static_cast<T>(s);
  }
  return o;
}

// GEO: kGeoMask (offsets [M][2T] + mask [M][T]), kGeoY (raw offset-conv output [M][3T],
// sigmoid of the mask part here), kGeoYF32 (the same from an fp32 y plus its fp32 bias) or
// kGeoRegular (no offsets: a plain convolution, used for the offset conv; fp32 bias and
// output). OutT: T, or float for the offset conv.
// TAPSTEP: C % BK == 0, so every K step lies inside one tap and a thread keeps its corner
// offsets and weights in registers from one tap to the next.
template <typename T, typename OutT, int BM, int BN, int BK, int WM_, int WN_, int GEO,
          bool TAPSTEP>
__global__ void __launch_bounds__(64 * WM_ * WN_) __attribute__((amdgpu_waves_per_eu(2, 8)))
dcn_fused_h_kernel(const HParams p) {
  constexpr int NT = 64 * WM_ * WN_, VEC = 8, KV = BK / VEC, KSUB = BK / 16;
  constexpr int AV = BM * KV / NT, LDA = BK + VEC;
  constexpr int WTM = BM / WM_, WTN = BN / WN_, TM = WTM / 32, TN = WTN / 32;
  static_assert(AV >= 1 && (BM * KV) % NT == 0 && TM >= 1 && TN >= 1, "tile config");
  using V = Vec<T, VEC>;
  __shared__ __attribute__((aligned(16))) TapGeo geo[BM * kMaxTaps];
  __shared__ __attribute__((aligned(16))) T As[2][BM * LDA];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN_, wn = wave - (wave / WN_) * WN_;
  // XCD x (= blockIdx % 8) runs tiles [x * tiles_per_xcd, (x + 1) * tiles_per_xcd)
  const int tile = (int)(blockIdx.x & 7) * p.tiles_per_xcd + (int)(blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= p.tiles_per_xcd || tile >= p.mt * p.nt) return;
  // K steps [ks0, ks1) of this workgroup (whole taps in the TAPSTEP form)
  const int nk = (p.K + BK - 1) / BK;
  const int ks0 = (int)blockIdx.y * p.kz_steps, ks1 = min(nk, ks0 + p.kz_steps);
  const int mtile = tile / p.nt;
  const int m0 = mtile * BM, n0 = (tile - mtile * p.nt) * BN;
  const int TT = p.taps;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  const uint32_t xoob = p.x_bytes, woob = p.w_bytes;

  // ---- geometry table -------------------------------------------------------------
  for (int g = tid; g < BM * TT; g += NT) {
    const int row = g / TT, t = g - row * TT, m = m0 + row;
    geo[g] = m < p.M ? tap_geo<T, GEO>(p, p.off, m, m, t) : empty_geo(xoob);
  }
  __syncthreads();

  // ---- A slots: (row, 16-byte k-vector); 8 consecutive lanes share a pixel ---------
  int a_row[AV], a_kv[AV], a_t[AV], a_c[AV];
#pragma unroll
  for (int i = 0; i < AV; ++i) {
    const int a = tid + i * NT;
    a_row[i] = a / KV;
    a_kv[i] = a - (a / KV) * KV;
    const int k = ks0 * BK + a_kv[i] * VEC;
    a_t[i] = k / p.C;
    a_c[i] = k - a_t[i] * p.C;
  }
  const int spt = TAPSTEP ? p.C / BK : 1;   // K steps per tap
  V ra[AV][4];
  float rw[AV][4];
  float gw[AV][4];      // TAPSTEP: weights and corner offsets of the current tap
  uint32_t go[AV][4];
  auto issue_a = [&](int ks) {
    if constexpr (TAPSTEP) {
      const int t = ks / spt, cstep = ks - t * spt;
      if (cstep == 0) {
#pragma unroll
        for (int i = 0; i < AV; ++i) {
          TapGeo G;
          if (t < TT) {
            G = geo[a_row[i] * TT + t];
          } else {
            G.w[0] = G.w[1] = G.w[2] = G.w[3] = 0.f;
            G.o[0] = G.o[1] = G.o[2] = G.o[3] = xoob;
          }
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            gw[i][q] = G.w[q];
            go[i][q] = G.o[q] == xoob ? xoob : G.o[q] + (uint32_t)(a_kv[i] * VEC) * (uint32_t)sizeof(T);
          }
        }
      }
      // channel offset of this step is uniform: it goes into the scalar offset
      const uint32_t so = (uint32_t)(cstep * BK) * (uint32_t)sizeof(T);
      constexpr int NQ = GEO == kGeoRegular ? 1 : 4;   // a plain conv reads one pixel
#pragma unroll
      for (int i = 0; i < AV; ++i)
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          rw[i][q] = gw[i][q];
          ra[i][q] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(xr, go[i][q], so, 0));
        }
    } else {
#pragma unroll
      for (int i = 0; i < AV; ++i) {
        if (ks > ks0) {
          a_c[i] += BK;
          while (a_c[i] >= p.C) { a_c[i] -= p.C; ++a_t[i]; }
        }
        TapGeo G;
        if (a_t[i] < TT) {
          G = geo[a_row[i] * TT + a_t[i]];
        } else {  // K tail
          G.w[0] = G.w[1] = G.w[2] = G.w[3] = 0.f;
          G.o[0] = G.o[1] = G.o[2] = G.o[3] = xoob;
        }
        const uint32_t cb = (uint32_t)a_c[i] * (uint32_t)sizeof(T);
        constexpr int NQ = GEO == kGeoRegular ? 1 : 4;
#pragma unroll
        for (int q = 0; q < NQ; ++q) {
          rw[i][q] = G.w[q];
          ra[i][q] = buffer_load_vec<T, VEC>(xr, G.o[q] == xoob ? xoob : G.o[q] + cb);
        }
      }
    }
  };
  // B: the block row of fragment column nb starts at bvo[j]; the K block goes into the
  // scalar offset. An absent column (N tail) gets an offset past the buffer and reads 0.
  int4v breg[2][KSUB][TN];
  uint32_t bvo[TN];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int nb = (n0 >> 5) + wn * TN + j;
    bvo[j] = nb < p.nb_total ? ((uint32_t)(nb * p.kb_total) * 64u + (uint32_t)lane) * 16u : woob;
  }
  auto issue_b = [&](int ks, int4v (&br)[KSUB][TN]) {
    if (ks * KSUB + KSUB <= p.kb_total) {
#pragma unroll
      for (int kk = 0; kk < KSUB; ++kk)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          br[kk][j] = __builtin_amdgcn_raw_buffer_load_b128(
              wr, bvo[j], (uint32_t)(ks * KSUB + kk) * 1024u, 0);
    } else {  // K tail: blocks past kb_total read 0
#pragma unroll
      for (int kk = 0; kk < KSUB; ++kk)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int kb = ks * KSUB + kk;
          br[kk][j] = __builtin_amdgcn_raw_buffer_load_b128(
              wr, kb < p.kb_total ? bvo[j] : woob, kb < p.kb_total ? (uint32_t)kb * 1024u : 0u, 0);
        }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int i = 0; i < AV; ++i) {
      V o;
      if constexpr (GEO == kGeoRegular) {
        o = ra[i][0];  // weight 1 on the one in-range pixel; 0 (read as 0) outside
      } else {
        o = blend4<T>(ra[i], rw[i][0], rw[i][1], rw[i][2], rw[i][3]);
      }
      store_vec<T, VEC>(&As[buf][a_row[i] * LDA + a_kv[i] * VEC], o);
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  const int lrow = lane & 31, lk = (lane >> 5) * 8;
  auto compute = [&](int buf, const int4v (&br)[KSUB][TN]) {
#pragma unroll
    for (int kk = 0; kk < KSUB; ++kk)
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const T *a = &As[buf][(wm * WTM + i * 32 + lrow) * LDA + kk * 16 + lk];
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16<T>(a, br[kk][j], acc[i][j]);
      }
  };

  // ---- K loop: A(k+1) is gathered and B(k+1) loaded while step k multiplies ---------
  // Pairs of steps with no exit in the middle of the body (an exit there makes the
  // compiler keep two copies of the accumulators), then an odd last step.
  issue_b(ks0, breg[0]);
  issue_a(ks0);
  store_a(0);
  if (ks0 + 1 < ks1) issue_a(ks0 + 1);
  int ks = ks0;
  for (; ks + 1 < ks1; ks += 2) {
    __syncthreads();                       // A(ks) complete in buffer 0
    issue_b(ks + 1, breg[1]);
    compute(0, breg[0]);
    store_a(1);                            // A(ks+1) -> buffer 1
    if (ks + 2 < ks1) issue_a(ks + 2);
    __syncthreads();
    if (ks + 2 < ks1) issue_b(ks + 2, breg[0]);
    compute(1, breg[1]);
    if (ks + 2 < ks1) {
      store_a(0);                          // A(ks+2) -> buffer 0
      if (ks + 3 < ks1) issue_a(ks + 3);
    }
  }
  if (ks < ks1) {
    __syncthreads();
    compute(0, breg[0]);
  }

  // ---- epilogue: lane holds col = lane % 32, rows 8*(e/4) + 4*(lane/32) + e%4 --------
  //      K in two parts (fp32 output): each adds its sum to the cleared output, the bias
  //      with the first; with two parts the result does not depend on their order.
  OutT *out = static_cast<OutT *>(p.out);
  using BiasT = typename std::conditional<GEO == kGeoRegular, float, T>::type;
  const BiasT *bias = static_cast<const BiasT *>(p.bias);
  const bool split = gridDim.y > 1;
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int n = n0 + (wn * TN + j) * 32 + lrow;
    const float bv = (bias != nullptr && n < p.Cout && blockIdx.y == 0) ? (float)bias[n] : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * WTM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        float v = acc[i][j][e] + bv;
        if (GEO != kGeoRegular && p.relu) v = v < 0.f ? 0.f : v;  // NaN stays NaN
        if (m < p.M && n < p.Cout) {
          if constexpr (std::is_same<OutT, float>::value) {
            if (split) unsafeAtomicAdd(out + (int64_t)m * p.Cout + n, v);
            else out[(int64_t)m * p.Cout + n] = v;
          } else {
            out[(int64_t)m * p.Cout + n] = static_cast<OutT>(v);
          }
        }
      }
  }
}

// Weight -> fragment blocks [NB][KB][64 lanes][8 elements]: lane l of block (nb, kb)
// holds W[n = nb*32 + l%32][k = kb*16 + (l/32)*8 + e], k = t*C + c, zero outside
// [0, Cout) x [0, K). Source layout [Cout][C][T] (module weight) or, with src_tc,
// [Cout][T][C]. One thread per 16-byte output chunk.
__global__ void __launch_bounds__(256) pack_weight_frag_kernel(const uint16_t *__restrict__ w,
                                                               uint16_t *__restrict__ packed,
                                                               int cout, int C, int T, int KB,
                                                               int64_t chunks, bool src_tc) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int64_t blk = i >> 6;
  const int l = (int)(i & 63);
  const int nb = (int)(blk / KB), kb = (int)(blk - (blk / KB) * KB);
  const int n = nb * 32 + (l & 31), k0 = kb * 16 + (l >> 5) * 8;
  const int K = C * T;
  Vec<uint16_t, 8> v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = k0 + e;
    const int t = k / C, c = k - (k / C) * C;
    const int64_t src = src_tc ? ((int64_t)n * T + t) * C + c : ((int64_t)n * C + c) * T + t;
    v.v[e] = (n < cout && k < K) ? w[src] : (uint16_t)0;
  }
  store_vec<uint16_t, 8>(packed + i * 8, v);
}

// Weight [Cout][T][C] (src_tc) with K % 8 == 0 -> fragment blocks: a chunk's 8 values are
// consecutive in the source row, one 16-byte load each.
__global__ void __launch_bounds__(256) pack_weight_frag_tc_kernel(const uint16_t *__restrict__ w,
                                                                  uint16_t *__restrict__ packed,
                                                                  int cout, int K, int KB,
                                                                  int64_t chunks) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= chunks) return;
  const int64_t blk = i >> 6;
  const int l = (int)(i & 63);
  const int nb = (int)(blk / KB), kb = (int)(blk - (blk / KB) * KB);
  const int n = nb * 32 + (l & 31), k0 = kb * 16 + (l >> 5) * 8;
  Vec<uint16_t, 8> v;
  if (n < cout && k0 < K) {
    v = load_vec<uint16_t, 8>(w + (int64_t)n * K + k0);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v.v[e] = 0;
  }
  store_vec<uint16_t, 8>(packed + i * 8, v);
}

// Weight [Cout][C][T] -> fragment blocks through LDS (C % 16 == 0, T <= kPackMaxT).
// Workgroup (nb, cg) takes the 32 rows of column block nb and channels [16 cg, 16 cg + 16)
// of every tap: each row's source span w[n][16 cg .. + 16)[0 .. T) is contiguous (16-byte
// loads), and the group's T K blocks (one per tap) are written from LDS as whole 16-byte
// chunks. The per-element form reads 8 values 2 T bytes apart for every chunk (res5: 14 us).
constexpr int kPackMaxT = 25;
__global__ void __launch_bounds__(256) pack_weight_frag_lds_kernel(const uint16_t *__restrict__ w,
                                                                   uint16_t *__restrict__ packed,
                                                                   int cout, int C, int T,
                                                                   int KB) {
  __shared__ __attribute__((aligned(16))) uint16_t s[32 * (16 * kPackMaxT + 8)];
  const int nb = (int)blockIdx.x, c0 = (int)blockIdx.y * 16;
  const int pitch = 16 * T + 8;  // elements per LDS row (16-byte multiple)
  const int vrow = 2 * T;        // 16-byte vectors per row span (16 T elements)
  for (int i = threadIdx.x; i < 32 * vrow; i += 256) {
    const int r = i / vrow, v = i - r * vrow, n = nb * 32 + r;
    Vec<uint16_t, 8> x;
    if (n < cout) {
      x = load_vec<uint16_t, 8>(w + ((int64_t)n * C + c0) * T + v * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x.v[e] = 0;
    }
    store_vec<uint16_t, 8>(&s[r * pitch + v * 8], x);
  }
  __syncthreads();
  for (int j = threadIdx.x; j < T * 64; j += 256) {
    const int l = j & 63, t = j >> 6;
    const int kb = (t * C + c0) >> 4;
    const int r = l & 31, cl = (l >> 5) * 8;
    Vec<uint16_t, 8> o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = s[r * pitch + (cl + e) * T + t];
    store_vec<uint16_t, 8>(packed + (((int64_t)nb * KB + kb) * 64 + l) * 8, o);
  }
}

// Weight [Cout][C][T] (or [Cout][T][C] with src_tc) -> [Cout][T][C] (fp32), one thread
// per output element.
__global__ void __launch_bounds__(256) pack_weight_kc_kernel(const float *__restrict__ w,
                                                             float *__restrict__ packed, int C,
                                                             int T, int64_t total, bool src_tc) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t n = i / ((int64_t)T * C);
  const int r = (int)(i - n * T * C), t = r / C, c = r - (r / C) * C;
  packed[i] = src_tc ? w[i] : w[(n * C + c) * T + t];
}

__global__ void __launch_bounds__(256) zero_f32_kernel(float *__restrict__ p, int64_t n) {
  const int64_t n4 = n >> 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256)
    reinterpret_cast<float4 *>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  const int64_t r = n4 * 4 + (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r < n) p[r] = 0.f;
}

// The offset conv of the usual DCN layer (3 x 3 taps, stride 1, dilation 1, C % 64 == 0,
// Cout <= 32) by output row segments: a workgroup takes 32 * NSUB (NSUB = 1, 2)
// consecutive pixels of one output row and loops over 64-channel chunks.
//   * A operand: per chunk the segment's input window (3 rows x 32 * NSUB + 2 pixels) is
//     staged in LDS once and every tap reads its fragments from it, so an input pixel
//     leaves L2 3 times instead of 9 (the tiled form gathers each tap separately).
//   * B operand: each wave loads its own weight fragments straight into registers; one
//     fragment feeds the MFMAs of all NSUB subtiles. Through LDS they would double the LDS
//     traffic, which (one 1 KB A fragment per 32 x 32 x 16 MFMA) already matches the
//     matrix cores' rate.
//   * Pipeline: while chunk c multiplies, chunk c + 1's window is written to the second
//     LDS buffer (one barrier per chunk) and chunk c + 3's window and chunk c + 2's
//     weights are loaded into registers.
//   * The chunk's 36 (tap, 16-channel block) MFMA steps are split over the 8 waves (wave w:
//     steps w, w + 8, ...); their partial sums meet in LDS and are added in wave order, so
//     every run gives the same result, with no atomics and no cleared output.
// Time is set by the latency of the chunk chain, not by bandwidth: B = 1 and B = 6 at the
// res5 shape measure alike (13.0 and 14.3 us, against 26.6 us plus a 4.8 us clear for the
// tiled form with K in two parts); at res4, 696 segments, one workgroup per CU, 27.4 us
// against 28.3 us.
constexpr int kBandWaves = 8, kBandPitch = 64 + 8;  // LDS window: halves per pixel
template <int NSUB> struct BandShape {
  static constexpr int SEG = 32 * NSUB, PW = SEG + 2;
  static constexpr int NU = (36 + kBandWaves - 1) / kBandWaves;  // MFMA steps per wave
  static constexpr int NV = 3 * PW * 8;                          // window vectors per chunk
  static constexpr int VPT = (NV + 64 * kBandWaves - 1) / (64 * kBandWaves);
  static constexpr int WIN_BYTES = 3 * PW * kBandPitch * 2;
  static constexpr int RED_BYTES = kBandWaves * NSUB * 1024 * 4;
  static constexpr int LDS = 2 * WIN_BYTES > RED_BYTES ? 2 * WIN_BYTES : RED_BYTES;
};

template <typename T, int NSUB>
__global__ void __launch_bounds__(64 * kBandWaves) offset_conv_band_kernel(const HParams p) {
  using S = BandShape<NSUB>;
  constexpr int NT = 64 * kBandWaves, NU = S::NU;
  static_assert(NSUB == 1 || NSUB == 2, "segment of one or two subtiles");
  using V = Vec<T, 8>;
  __shared__ __attribute__((aligned(16))) unsigned char smem[S::LDS];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // XCD x (= blockIdx % 8) runs segments [x * tiles_per_xcd, (x + 1) * tiles_per_xcd):
  // neighbouring output rows, whose windows overlap, share that XCD's L2
  const int idx = (int)(blockIdx.x & 7) * p.tiles_per_xcd + (int)(blockIdx.x >> 3);
  if ((int)(blockIdx.x >> 3) >= p.tiles_per_xcd || idx >= p.mt) return;
  const int row = idx / p.nt, ow0 = (idx - row * p.nt) * S::SEG;  // row = b * Ho + oh
  const int b = row / p.Ho, oh = row - b * p.Ho;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);

  // window slots: vector q (16 bytes) of pixel px of window row r; byte offset in x
  // (x_bytes outside the image: reads 0) and byte offset in an LDS buffer (-1: spare slot)
  uint32_t xo[S::VPT];
  int wl[S::VPT];
#pragma unroll
  for (int i = 0; i < S::VPT; ++i) {
    const int v = tid + i * NT;
    const int r = v / (S::PW * 8), rem = v - r * (S::PW * 8), px = rem >> 3, q = rem & 7;
    const int h = oh - p.ph + r, w = ow0 - p.pw + px;
    const bool in = v < S::NV && h >= 0 && h < p.H && w >= 0 && w < p.W;
    xo[i] = in ? (uint32_t)((b * p.H + h) * p.W + w) * (uint32_t)p.C * (uint32_t)sizeof(T) +
                     (uint32_t)q * 16u
               : p.x_bytes;
    wl[i] = v < S::NV ? ((r * S::PW + px) * kBandPitch + q * 8) * (int)sizeof(T) : -1;
  }
  // this wave's MFMA steps u = wave + 8 j (tap u / 4, 16-channel block u % 4; steps past
  // 35 load step 35 and skip the MFMA) and the lane's 16 bytes of their weight fragments:
  // block (tap * C + chunk * 64) / 16 + u % 4 of the packed weight
  uint32_t bo[NU];
#pragma unroll
  for (int j = 0; j < NU; ++j) {
    const int u = min(wave + j * kBandWaves, 35);
    bo[j] = (uint32_t)((u >> 2) * (p.C / 16) + (u & 3)) * 1024u + (uint32_t)lane * 16u;
  }

  // Chunk c's window is loaded into register stage c % 2 at step c - 3 and written to LDS
  // buffer c % 2 at step c - 1; its weights are loaded into stage c % 2 at step c - 2.
  // Every load is issued unconditionally (chunk indices past the end repeat the last
  // chunk), so the vector-memory wait counts are exact.
  const int nch = p.C / 64;
  V xv[2][S::VPT];
  int4v wb[2][NU];
  auto load_x = [&](V (&x)[S::VPT], int cc) {
    const uint32_t so = (uint32_t)min(cc, nch - 1) * 128u;
#pragma unroll
    for (int i = 0; i < S::VPT; ++i)
      x[i] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(xr, xo[i], so, 0));
  };
  auto load_w = [&](int4v (&w)[NU], int cc) {
    const uint32_t so = (uint32_t)min(cc, nch - 1) * 4096u;
#pragma unroll
    for (int j = 0; j < NU; ++j) w[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, bo[j], so, 0);
  };
  auto store_x = [&](const V (&x)[S::VPT], int buf) {
#pragma unroll
    for (int i = 0; i < S::VPT; ++i)
      if (wl[i] >= 0) *reinterpret_cast<V *>(smem + buf * S::WIN_BYTES + wl[i]) = x[i];
  };

  // lane's A fragment row: pixel 32 k + lane % 32 of subtile k, channels 8 (lane / 32) + ..
  const T *abase = reinterpret_cast<const T *>(smem) + (lane & 31) * kBandPitch + (lane >> 5) * 8;
  floatx16 acc[NSUB];
#pragma unroll
  for (int k = 0; k < NSUB; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
  // fragment f = (step j = f / NSUB, subtile k = f % NSUB), read RING fragments ahead of
  // its MFMA (left to itself the scheduler moves each read next to its MFMA)
  constexpr int NF = NU * NSUB, RING = 4;
  auto frag = [&](int f, int buf) -> int4v {
    const int j = f / NSUB, k = f - j * NSUB;
    const int u = min(wave + j * kBandWaves, 35), t = u >> 2, ki = t / 3, kj = t - ki * 3;
    return *reinterpret_cast<const int4v *>(abase + buf * (S::WIN_BYTES / (int)sizeof(T)) +
                                            (ki * S::PW + kj + 32 * k) * kBandPitch +
                                            (u & 3) * 16);
  };
  auto compute = [&](const int4v (&w)[NU], int buf) {
    int4v fa[RING];
#pragma unroll
    for (int f = 0; f < RING && f < NF; ++f) fa[f] = frag(f, buf);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      const int j = f / NSUB, k = f - j * NSUB;
      if (wave + j * kBandWaves < 36) acc[k] = mfma16r<T>(fa[f % RING], w[j], acc[k]);
      if (f + RING < NF) fa[f % RING] = frag(f + RING, buf);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  load_w(wb[0], 0);
  load_w(wb[1], 1);
  load_x(xv[0], 0);
  load_x(xv[1], 1);
  store_x(xv[0], 0);
  load_x(xv[0], 2);
  __syncthreads();
  // step cc: chunk cc + 1's window into the other buffer while chunk cc multiplies; steps
  // past the last chunk skip the MFMAs (an exit inside the unrolled pair would make the
  // compiler keep every stage twice)
#pragma nounroll
  for (int c0 = 0; c0 < nch; c0 += 2) {
#pragma unroll
    for (int d = 0; d < 2; ++d) {
      const int cc = c0 + d;
      store_x(xv[d ^ 1], d ^ 1);
      load_x(xv[d ^ 1], cc + 3);
      if (cc < nch) compute(wb[d], d);
      load_w(wb[d], cc + 2);
      __syncthreads();  // window cc + 1 complete, every wave done with window cc
    }
  }

  // partial sums: wave w's subtile k at red[(w * NSUB + k) * 1024 + e * 64 + lane], added
  // in wave order
  float *red = reinterpret_cast<float *>(smem);
#pragma unroll
  for (int k = 0; k < NSUB; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[(wave * NSUB + k) * 1024 + e * 64 + lane] = acc[k][e];
  __syncthreads();
  float *out = static_cast<float *>(p.out);
  const float *bias = static_cast<const float *>(p.bias);
  for (int o = tid; o < NSUB * 1024; o += NT) {
    const int k = o >> 10, r = o & 1023;
    float v = red[k * 1024 + r];
#pragma unroll
    for (int w = 1; w < kBandWaves; ++w) v += red[(w * NSUB + k) * 1024 + r];
    const int e = r >> 6, l = r & 63, n = l & 31;
    const int ow = ow0 + 32 * k + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
    if (ow < p.Wo && n < p.Cout) {
      if (bias != nullptr) v += bias[n];
      out[((int64_t)row * p.Wo + ow) * p.Cout + n] = v;
    }
  }
}

template <typename T, typename OutT, int BM, int BN, int BK, int WM, int WN, bool TAPSTEP>
hipError_t launch_cfg(HParams p, int geo, hipStream_t stream) {
  p.mt = (p.M + BM - 1) / BM;
  p.nt = (p.Cout + BN - 1) / BN;
  p.tiles_per_xcd = (p.mt * p.nt + 7) / 8;
  const int nk = (p.K + BK - 1) / BK;
  p.kz_steps = nk;
  // fp32 output (the offset conv) with fewer than two tiles per CU: K in two parts that
  // add into the cleared output, twice the K chains at once (res5 front end, 272 one-wave
  // tiles: 70.9 -> 60.7 us; res4, 1088 tiles, slows down, 75.6 -> 86.7 us, and stays whole).
  // The TAPSTEP form reads a tap's geometry at its first step, so a part is whole taps.
  const int spt = TAPSTEP ? p.C / BK : 1;
  const int units = TAPSTEP ? p.taps : nk;
  if (std::is_same<OutT, float>::value && units >= 2 && nk >= 16 &&
      (int64_t)p.mt * p.nt < 2 * (int64_t)device_cus() &&
      reinterpret_cast<uintptr_t>(p.out) % 16 == 0) {
    p.kz_steps = (units + 1) / 2 * spt;
    const int64_t n = (int64_t)p.M * p.Cout;
    const unsigned g = (unsigned)std::max<int64_t>(1, std::min<int64_t>((n / 4 + 255) / 256, 4096));
    hipLaunchKernelGGL(zero_f32_kernel, dim3(g), dim3(256), 0, stream, static_cast<float *>(p.out), n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const dim3 grid(8 * p.tiles_per_xcd, (nk + p.kz_steps - 1) / p.kz_steps), block(64 * WM * WN);
  if constexpr (std::is_same<OutT, float>::value) {  // fp32 output: the plain convolution only
    if (geo != kGeoRegular) return hipErrorInvalidValue;
    hipLaunchKernelGGL((dcn_fused_h_kernel<T, OutT, BM, BN, BK, WM, WN, kGeoRegular, TAPSTEP>),
                       grid, block, 0, stream, p);
    return hipGetLastError();
  } else {  // input-dtype output: the deformable forms
    if (geo == kGeoY)
      hipLaunchKernelGGL((dcn_fused_h_kernel<T, OutT, BM, BN, BK, WM, WN, kGeoY, TAPSTEP>), grid,
                         block, 0, stream, p);
    else if (geo == kGeoYF32)
      hipLaunchKernelGGL((dcn_fused_h_kernel<T, OutT, BM, BN, BK, WM, WN, kGeoYF32, TAPSTEP>),
                         grid, block, 0, stream, p);
    else if (geo == kGeoMask)
      hipLaunchKernelGGL((dcn_fused_h_kernel<T, OutT, BM, BN, BK, WM, WN, kGeoMask, TAPSTEP>),
                         grid, block, 0, stream, p);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
}

template <typename T, int NSUB>
hipError_t launch_band(HParams p, hipStream_t stream) {
  using S = BandShape<NSUB>;
  if (p.M == 0) return hipSuccess;
  p.nt = (p.Wo + S::SEG - 1) / S::SEG;  // segments per output row
  p.mt = (p.M / p.Wo) * p.nt;           // segments
  p.tiles_per_xcd = (p.mt + 7) / 8;
  hipLaunchKernelGGL((offset_conv_band_kernel<T, NSUB>), dim3(8 * p.tiles_per_xcd),
                     dim3(64 * kBandWaves), 0, stream, p);
  return hipGetLastError();
}

bool band_geometry(const HParams &p) {
  return p.kh == 3 && p.kw == 3 && p.sh == 1 && p.sw == 1 && p.dh == 1 && p.dw == 1 &&
         p.C % 64 == 0 && p.Cout <= 32;
}

template <typename T, bool TAPSTEP>
hipError_t launch_tt(const HParams &p, int geo, hipStream_t stream) {
  // Offset conv: Cout = 3T <= 27, fp32 output. One-wave 32 x 32 tiles: no wave spends
  // the K loop on columns past Cout, and the K chain of each tile (the bound: the work per
  // step is small) runs in twice as many tiles at once (res4 front end 85 -> 82 us against
  // 64 x 64 tiles of 4 waves). K steps of 128 channels where C allows halve the chain's
  // length (front end res4 75.6 -> 73.9 us, res5 60.9 -> 55.5 us; 256 channels, 254
  // registers and 42 KB of LDS, measured 86.7 and 57.6 us).
  if (geo == kGeoRegular) {
    if (TAPSTEP && band_geometry(p))
      return p.Wo > 32 ? launch_band<T, 2>(p, stream) : launch_band<T, 1>(p, stream);
    if (TAPSTEP && p.C % 128 == 0)
      return launch_cfg<T, float, 32, 32, 128, 1, 1, true>(p, geo, stream);
    return launch_cfg<T, float, 32, 32, 64, 1, 1, TAPSTEP>(p, geo, stream);
  }
  if (p.Cout > 128) return launch_cfg<T, T, 64, 256, 64, 1, 4, TAPSTEP>(p, geo, stream);
  if (p.Cout > 64) return launch_cfg<T, T, 64, 128, 64, 2, 2, TAPSTEP>(p, geo, stream);
  return launch_cfg<T, T, 64, 64, 64, 2, 2, TAPSTEP>(p, geo, stream);
}

// ---------------------------------------------------------------------------------------
// Persistent, row-balanced variant (128 < Cout <= 512, C % 64 == 0), for row chunks of at
// most 5 blocks (80-row tiles; larger chunks run dcn_fused_s_kernel). One workgroup of 8
// waves per CU owns contiguous chunks of 16-row blocks of M (p_config_for) and all BN = 256
// output channels of one column half for the whole K loop. The waves specialise: waves
// 0-3 ("consumers") run the MFMAs, wave c
// computing columns [64 c, 64 c + 64) of every row block with v_mfma_f32_16x16x32 and
// loading its B fragments from the fragment-packed weight one step ahead; waves 4-7
// ("producers") gather the four corners of every (row, 16-byte k-vector) slot two steps
// ahead into two register sets, blend them (bilinear x mask weights) and write the A
// tile of the next step into a double-buffered LDS tile. A workgroup's waves are spread
// round-robin over the CU's four SIMDs, so every SIMD runs one consumer and one producer:
// the matrix core works while the other wave's gathers and blend math proceed. One
// barrier per K step (64 channels of one tap) hands the A tile over. The row range is
// XCD-contiguous (XCD x owns the x-th eighth of M), so the image rows its gathers touch
// stay in that XCD's L2.
constexpr int kPBK = 64, kPLDA = kPBK;          // K step, A tile row pitch (elements)

// A tile element offset of (row, 16-byte chunk of the K step): rows are 128 bytes and the
// chunk index is XORed with (row / 2) % 8, so the producers' stores (two rows of eight
// chunks per 16 lanes) and the consumers' fragment reads (16 rows, one chunk) each touch
// 16 distinct 16-byte bank groups.
__device__ __forceinline__ int a_off(int row, int chunk) {
  return row * kPLDA + ((chunk ^ ((row >> 1) & 7)) << 3);
}
constexpr int kPKH = kPBK / 32;                 // 16x16x32 MFMA k-blocks per step
constexpr int kPThreads = 512;                  // 4 consumer + 4 producer waves
constexpr int kPProd = 256;                     // producer threads
constexpr int kPCols = 256;                     // output columns per workgroup
constexpr int kPStage = kPCols + 8;             // output staging row pitch (elements)

// Workgroup shape for NRB 16-row blocks (at most; a workgroup stores NRB - 1 or NRB).
template <int NRB>
struct PShape {
  static constexpr int kRows = NRB * 16;
  static constexpr int kSlots = kRows * (kPBK / 8);  // (row, 16-byte k-vector) slots per step
  static constexpr int kSPT = (kSlots + kPProd - 1) / kPProd;  // slots per producer thread
  static constexpr int kLastWaves = (kSlots - (kSPT - 1) * kPProd) / kWave;
  static_assert(kLastWaves * kWave == kSlots - (kSPT - 1) * kPProd && kLastWaves >= 1,
                "the last slot set must cover whole producer waves");
  // K steps in flight: gathers (producers) and weight fragments (consumers). Few rows
  // leave a step little work to cover a gather's round trip, and registers to spare.
  static constexpr int kPD = NRB <= 3 ? 6 : 2;
  static constexpr int kCD = NRB <= 3 ? 4 : 2;
};

typedef float floatx4 __attribute__((ext_vector_type(4)));

template <typename T> __device__ __forceinline__ floatx4 mfma16x16(int4v a, int4v b, floatx4 c);
template <> __device__ __forceinline__ floatx4 mfma16x16<f16>(int4v a, int4v b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a),
                                                __builtin_bit_cast(half8, b), c, 0, 0, 0);
}
template <> __device__ __forceinline__ floatx4 mfma16x16<bf16>(int4v a, int4v b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

struct PParams {
  HParams h;
  int rb_total;  // 16-row blocks of M
  int nblocks;   // workgroups resident at once, one per CU (a multiple of 8)
  int halves;    // 256-column halves of Cout (1 or 2): XCDs 0-3 take half 0, 4-7 half 1
  int rounds;    // the grid is nblocks * rounds workgroups, one row chunk each: each
                 // half's blocks are cut into rounds * nblocks / halves balanced chunks of
                 // at most NRB blocks
};

// B fragment of v_mfma_f32_16x16x32 read from the 32x32x16 fragment packing: lane l takes
// column n and k = 32 kh + 8 (l >> 4) .. + 8 of a K step, i.e. block (n / 32, 2 kh +
// (l >> 5)), lane (n % 32) + 32 ((l >> 4) & 1) of the packing.
__device__ __forceinline__ uint32_t b_frag_offset(int n, int kh, int lane, int nb_total,
                                                  int kb_total, uint32_t oob) {
  const int nb = n >> 5;
  return nb < nb_total ? ((uint32_t)(nb * kb_total + 2 * kh + (lane >> 5)) * 64u +
                          (uint32_t)((n & 31) + 32 * ((lane >> 4) & 1))) * 16u
                       : oob;
}

// Consumer wave c: B(k+2) issued at step k, MFMA(k) from A buffer k % 2, one barrier per
// step; then the epilogue (bias, relu, one rounding) into the LDS output tile `stage`,
// which the whole workgroup stores afterwards as full 16-byte pieces of output rows.
// Always NRB row blocks (compile-time, so the MFMA loop and the accumulators carry no
// run-time conditions).
template <typename T, int NRB, int CD>
__device__ __forceinline__ void dcn_p_consumer(const HParams &p, T (*As)[NRB * 16 * kPLDA],
                                               T *stage, int n0, int nk, int lane, int wave,
                                               const int4v (&b0)[kPKH][4], bool b0_loaded) {
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  uint32_t bo[kPKH][4];
#pragma unroll
  for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
      bo[kh][cb] = b_frag_offset(n0 + wave * 64 + cb * 16 + (lane & 15), kh, lane, p.nb_total,
                                 p.kb_total, p.w_bytes);
  auto issue_b = [&](int ks, int4v (&br)[kPKH][4]) __attribute__((always_inline)) {
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        br[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(
            wr, bo[kh][cb], (uint32_t)ks * (uint32_t)(kPBK / 16) * 1024u, 0);
  };
  floatx4 acc[NRB][4];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  // CD B register sets: B(k+CD) is loaded right after step k's MFMAs, so a weight load
  // queued behind the producers' gathers has CD - 1 steps to arrive.
  int4v br[CD][kPKH][4];
  auto step = [&](int ks, int4v (&br)[kPKH][4]) __attribute__((always_inline)) {
    const int buf = ks & 1;
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh) {
      int4v af[NRB];
#pragma unroll
      for (int rbi = 0; rbi < NRB; ++rbi)
        af[rbi] = *reinterpret_cast<const int4v *>(
            &As[buf][a_off(rbi * 16 + (lane & 15), kh * 4 + (lane >> 4))]);
#pragma unroll
      for (int rbi = 0; rbi < NRB; ++rbi)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb)
          acc[rbi][cb] = mfma16x16<T>(af[rbi], br[kh][cb], acc[rbi][cb]);
    }
    issue_b(ks + CD, br);
    __syncthreads();
  };
  if (b0_loaded) {  // B(0) loaded by the caller before the geometry table
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) br[0][kh][cb] = b0[kh][cb];
  } else {
    issue_b(0, br[0]);
  }
#pragma unroll
  for (int d = 1; d < CD; ++d) issue_b(d, br[d]);
  __syncthreads();  // A(0) written by the producers
  int ks = 0;
  for (; ks + CD <= nk; ks += CD) {
#pragma unroll
    for (int d = 0; d < CD; ++d) step(ks + d, br[d]);
  }
#pragma unroll
  for (int d = 0; d + 1 < CD; ++d)
    if (ks + d < nk) step(ks + d, br[d]);

  // Epilogue: lane holds column 64 wave + 16 cb + (lane & 15), rows 4 (lane >> 4) + e.
  const T *bias = static_cast<const T *>(p.bias);
#pragma unroll
  for (int cb = 0; cb < 4; ++cb) {
    const int c = wave * 64 + cb * 16 + (lane & 15);
    const float bv = (bias != nullptr && n0 + c < p.Cout) ? (float)bias[n0 + c] : 0.f;
#pragma unroll
    for (int rbi = 0; rbi < NRB; ++rbi)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[rbi][cb][e] + bv;
        if (p.relu) v = v < 0.f ? 0.f : v;  // NaN stays NaN, as torch.relu
        stage[(rbi * 16 + 4 * (lane >> 4) + e) * kPStage + c] = static_cast<T>(v);
      }
  }
}

// Offset conv of the one-launch forward, consumer side: y[row][n] = sum_k A[row, k] *
// Woff[n, k] + b_off[n] for the workgroup's NRB * 16 rows and n < 32 (3T <= 27 used), in
// fp32. Wave c takes the row blocks c, c + 4, c + 8 (a block past NRB repeats the last
// one and is not stored, so no MFMA is conditional) and both 16-column blocks; every wave
// loads the same B fragments (4 per step). At the end y goes to ys (LDS, row pitch 3T) and
// to p.y_out when that is given. Same barrier sequence as dcn_p_consumer.
template <typename T, int NRB>
__device__ __forceinline__ void dcn_p_offset_consumer(const HParams &p,
                                                      T (*As)[NRB * 16 * kPLDA], float *ys,
                                                      int m0, int nrb, int nk, int lane,
                                                      int wave) {
  constexpr int RB = (NRB + 3) / 4;
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w2, p.w2_bytes);
  const int kb2 = p.K / 16;
  uint32_t bo[kPKH][2];
#pragma unroll
  for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      bo[kh][cb] = b_frag_offset(cb * 16 + (lane & 15), kh, lane, 1, kb2, p.w2_bytes);
  auto issue_b = [&](int ks, int4v (&br)[kPKH][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        br[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(
            wr, bo[kh][cb], (uint32_t)ks * (uint32_t)(kPBK / 16) * 1024u, 0);
  };
  floatx4 acc[RB][2];
#pragma unroll
  for (int i = 0; i < RB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  int4v br[kPKH][2];
  issue_b(0, br);
  __syncthreads();  // A(0) written by the producers
  for (int ks = 0; ks < nk; ++ks) {
    const int buf = ks & 1;
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh) {
      int4v af[RB];
#pragma unroll
      for (int i = 0; i < RB; ++i) {
        const int rb = min(wave + 4 * i, NRB - 1);
        af[i] = *reinterpret_cast<const int4v *>(
            &As[buf][a_off(rb * 16 + (lane & 15), kh * 4 + (lane >> 4))]);
      }
#pragma unroll
      for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) acc[i][cb] = mfma16x16<T>(af[i], br[kh][cb], acc[i][cb]);
    }
    issue_b(ks + 1, br);
    __syncthreads();
  }
  // The last barrier above ends every read and write of the A ring: ys may alias it.
  const int n3 = 3 * p.taps;
#pragma unroll
  for (int i = 0; i < RB; ++i) {
    const int rb = wave + 4 * i;
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int n = cb * 16 + (lane & 15);
      const float bv = (n < n3 && p.b2 != nullptr) ? p.b2[n] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = rb * 16 + 4 * (lane >> 4) + e;
        if (rb < nrb && n < n3) {
          const float v = acc[i][cb][e] + bv;
          ys[row * n3 + n] = v;
          if (p.y_out != nullptr && m0 + row < p.M) p.y_out[(int64_t)(m0 + row) * n3 + n] = v;
        }
      }
    }
  }
}

// Producer thread ptid (0..255) with NS gather slots: slot i is (row, k-vector) =
// (s / KV, s % KV), s = ptid + 256 i. The gathers of step k + PD are issued at step k into
// register set k % PD (blended at step k - 1); A(k+1) is blended at step k from set
// (k+1) % PD into buffer (k+1) % 2. Every load is issued unconditionally (steps past the
// end read out of range), so the compiler's wait counts stay exact and the gathers of the
// next steps stay in flight. REG: plain convolution taps (one pixel per slot, no blend).
template <typename T, int NS, int NRB, bool REG, int PD>
__device__ __forceinline__ void dcn_p_producer(const HParams &p, const TapGeo *geo,
                                               T (*As)[NRB * 16 * kPLDA], int nk, int ptid) {
  using V = Vec<T, 8>;
  constexpr int KV = kPBK / 8;
  constexpr int NQ = REG ? 1 : 4;
  const int TT = p.taps;
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const uint32_t xoob = p.x_bytes;
  const int kv = ptid % KV;
  const int spt = p.C / kPBK;  // K steps per tap
  uint32_t go[NS][NQ];         // corner offsets of the tap being issued (+ k-vector)
  auto load_geo = [&](int t) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      if (t < TT) {
        const TapGeo &G = geo[((ptid + i * kPProd) / KV) * TT + t];
#pragma unroll
        for (int q = 0; q < NQ; ++q)
          go[i][q] = G.o[q] == xoob ? xoob : G.o[q] + (uint32_t)(kv * 8 * sizeof(T));
      } else {
#pragma unroll
        for (int q = 0; q < NQ; ++q) go[i][q] = xoob;
      }
    }
  };
  auto issue_gather = [&](int ks, V (&ra)[NS][NQ]) __attribute__((always_inline)) {
    const int t = ks / spt, cs = ks - t * spt;
    if (cs == 0) load_geo(t);
    const uint32_t so = (uint32_t)(cs * kPBK * sizeof(T));
#pragma unroll
    for (int i = 0; i < NS; ++i)
#pragma unroll
      for (int q = 0; q < NQ; ++q)
        ra[i][q] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(xr, go[i][q], so, 0));
  };
  auto blend = [&](int ks, const V (&ra)[NS][NQ], int buf) __attribute__((always_inline)) {
    // Past the last step the gathered corners are zero (out-of-range offsets); the tap is
    // clamped so the weight read stays inside the table.
    const int t = min(ks / spt, TT - 1);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
      const int row = (ptid + i * kPProd) / KV;
      V o;
      if constexpr (REG) {
        o = ra[i][0];  // the in-image pixel, or zeros read out of range
      } else {
        const float4 w = *reinterpret_cast<const float4 *>(geo[row * TT + t].w);
        o = blend4<T>(ra[i], w.x, w.y, w.z, w.w);
      }
      store_vec<T, 8>(&As[buf][a_off(row, kv)], o);
    }
  };
  V ra[PD][NS][NQ];
  auto step = [&](int ks, V (&ra_issue)[NS][NQ], const V (&ra_blend)[NS][NQ])
      __attribute__((always_inline)) {
    issue_gather(ks + PD, ra_issue);
    blend(ks + 1, ra_blend, (ks + 1) & 1);
    __syncthreads();
  };
#pragma unroll
  for (int d = 0; d < PD; ++d) issue_gather(d, ra[d]);
  blend(0, ra[0], 0);
  __syncthreads();
  int k0 = 0;
  for (; k0 + PD <= nk; k0 += PD) {
#pragma unroll
    for (int d = 0; d < PD; ++d) step(k0 + d, ra[d], ra[(d + 1) % PD]);
  }
#pragma unroll
  for (int d = 0; d + 1 < PD; ++d)
    if (k0 + d < nk) step(k0 + d, ra[d], ra[(d + 1) % PD]);
}

// GEO: kGeoMask, kGeoY or kGeoYF32 (read from global memory). MEGA: the one-launch
// forward; a first pass over K computes the offset conv of the workgroup's rows on the
// matrix cores (dcn_p_offset_consumer + plain-convolution producers), its fp32 output
// with bias is kept in LDS (aliasing the A ring) and the deformable geometry is built from
// it, as the reference's single-kernel forward does (fused_tl.py:565-688).
template <typename T, int GEO, int NRB, bool MEGA>
__global__ void __launch_bounds__(kPThreads) dcn_fused_p_kernel(const PParams pp) {
  using SH = PShape<NRB>;
  constexpr int kPRows = SH::kRows;
  const HParams &p = pp.h;
  __shared__ __attribute__((aligned(16))) TapGeo geo[kPRows * kMaxTaps];
  __shared__ __attribute__((aligned(16))) T As[2][kPRows * kPLDA];
  __shared__ __attribute__((aligned(16))) T stage[kPRows * kPStage];  // the output tile
  static_assert(!MEGA || sizeof(As) >= sizeof(float) * kPRows * 3 * kMaxTaps,
                "the offset-conv output must fit in the A ring");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Workgroup b runs on XCD b % 8; XCD x takes a contiguous range of its half's chunks, so
  // the image rows its gathers touch stay in its L2. With two column halves XCDs 0-3 take
  // half 0 and 4-7 half 1, so each XCD's L2 holds one half of the weight.
  const int bpx = (int)(gridDim.x >> 3);               // workgroups per XCD
  const int xcd = (int)(blockIdx.x & 7);
  const int xph = 8 / pp.halves;                       // XCDs per half
  const int half = xcd / xph;
  const int nch = (int)gridDim.x / pp.halves;          // row chunks per half
  const int j = (xcd - half * xph) * bpx + (int)(blockIdx.x >> 3);
  const int n0 = half * kPCols;
  const int TT = p.taps;
  const uint32_t xoob = p.x_bytes;
  const int nk = TT * (p.C / kPBK);
  float *ys = reinterpret_cast<float *>(&As[0][0]);
  const int rb0 = (int)((int64_t)pp.rb_total * j / nch);
  const int nrb = (int)((int64_t)pp.rb_total * (j + 1) / nch) - rb0;  // at most NRB
  if (nrb <= 0) return;
  const int m0 = rb0 * 16;
  const int nrows = nrb * 16;

  if constexpr (MEGA) {
    // Pass 1: the offset conv. Plain-convolution geometry (one pixel per row and tap).
    for (int g = tid; g < kPRows * TT; g += kPThreads) {
      const int row = g / TT, t = g - row * TT, m = m0 + row;
      geo[g] = (row < nrows && m < p.M) ? tap_geo<T, kGeoRegular>(p, nullptr, 0, m, t)
                                        : empty_geo(xoob);
    }
    __syncthreads();
    if (wave < 4)
      dcn_p_offset_consumer<T, NRB>(p, As, ys, m0, nrb, nk, lane, wave);
    else if (wave - 4 < SH::kLastWaves)
      dcn_p_producer<T, SH::kSPT, NRB, true, 2>(p, geo, As, nk, tid - kPProd);
    else if constexpr (SH::kLastWaves < 4)
      dcn_p_producer<T, SH::kSPT - 1, NRB, true, 2>(p, geo, As, nk, tid - kPProd);
    __syncthreads();  // y of every row in ys
  }

  // The consumers' B fragments of K step 0, loaded before the geometry table (they do not
  // need it) where the consumers keep two B sets (4-5 row blocks): res5 fp16 74.1 -> 71.7 us,
  // bf16 74.4 -> 74.1 us, res5 one-launch fp16 84.6 -> 83.0 us. Loading both sets early
  // measured res5 bf16 74.2 -> 75.0 us, and with four sets (2-3 row blocks) it spills.
  constexpr bool kB0Early = SH::kCD == 2;
  int4v b0[kPKH][4];
  if (kB0Early && wave < 4) {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 4; ++cb)
        b0[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(
            wr, b_frag_offset(n0 + wave * 64 + cb * 16 + (lane & 15), kh, lane, p.nb_total,
                              p.kb_total, p.w_bytes), 0u, 0);
  }
  // Geometry table for all NRB * 16 rows (rows outside the range or past M: zero weights,
  // out-of-range offsets).
  for (int g = tid; g < kPRows * TT; g += kPThreads) {
    const int row = g / TT, t = g - row * TT, m = m0 + row;
    TapGeo G = empty_geo(xoob);
    if (row < nrows && m < p.M) {
      if constexpr (MEGA)
        G = tap_geo<T, kGeoYF32>(p, ys, row, m, t);   // bias already in ys
      else
        G = tap_geo<T, GEO>(p, p.off, m, m, t);
    }
    geo[g] = G;
  }
  __syncthreads();  // MEGA: ys is dead from here, the A ring is written again
  // Always the NRB-block body: a range of NRB - 1 blocks has zero geometry in its last
  // block (see above) and does not store it; the kernel's time is set by the full ranges.
  // Consumers and producers run the same number of barriers (one per step + prologue).
  // Producer waves issue first when both roles are ready: the gathers of the next K step
  // leave earlier and the matrix-core work waits less at the barrier (res4 fp16 71.0 ->
  // 67.8 us; the consumers raised instead, 70.2 us).
  if (wave >= 4) __builtin_amdgcn_s_setprio(2);
  if (wave < 4)
    dcn_p_consumer<T, NRB, SH::kCD>(p, As, stage, n0, nk, lane, wave, b0, kB0Early);
  else if (wave - 4 < SH::kLastWaves)
    dcn_p_producer<T, SH::kSPT, NRB, false, SH::kPD>(p, geo, As, nk, tid - kPProd);
  else if constexpr (SH::kLastWaves < 4)
    dcn_p_producer<T, SH::kSPT - 1, NRB, false, SH::kPD>(p, geo, As, nk, tid - kPProd);
  // The output tile: full 16-byte pieces of the workgroup's rows (Cout % 8 == 0 and a
  // 16-byte aligned output, checked on the host: a piece is wholly inside or outside),
  // streaming stores (written once; the input rows stay in L2).
  __syncthreads();
  T *out = static_cast<T *>(p.out);
  constexpr int kPieces = kPCols / 8;
  for (int i = tid; i < nrows * kPieces; i += kPThreads) {
    const int row = i / kPieces, c = (i - row * kPieces) * 8, m = m0 + row;
    if (m < p.M && n0 + c < p.Cout)
      __builtin_nontemporal_store(*reinterpret_cast<const int4v *>(&stage[row * kPStage + c]),
                                  reinterpret_cast<int4v *>(out + (int64_t)m * p.Cout + n0 + c));
  }
}

// ---------------------------------------------------------------------------------------
// Symmetric persistent kernel (fp16 / bf16, 128 < Cout <= 512, C % 64 == 0): the work
// split of dcn_fused_p_kernel (one workgroup per CU, NRB 16-row blocks x one 256-column
// half of Cout, XCD-contiguous row ranges) with eight waves that each do both jobs:
//   * MFMA: wave w computes columns [32 w, 32 w + 32) of every row block
//     (v_mfma_f32_16x16x32) from the A tile in LDS, its A fragments read kSAhead
//     fragments ahead in a fixed order, its B fragments loaded two steps ahead;
//   * gather: thread t owns the A-tile slots (row t / 8 + 64 i, 16-byte k-vector t % 8)
//     with one register set of corners per slot; at step k it blends the slot's corners
//     of step k + 1 into the other A buffer and issues the slot's loads of step k + 2.
// Why this split (measured on gfx950): one wave issues vector ALU instructions at about
// one per 8 cycles while two waves on a SIMD reach one per 4, so the blend arithmetic
// (about 250 instructions per SIMD and K step) runs twice as fast spread over both waves
// of each SIMD as on one producer wave; and a wave with about one step of gathers in
// flight (8-12 loads here) keeps the vector-memory path busier than one with two steps
// (about 40 loads). The price is that every wave reads the whole A tile from LDS.
// One barrier per K step (64 channels of one tap) hands the A tile over.
constexpr int kSThreads = 512;
constexpr int kSAhead = 3;  // A fragments read ahead of their MFMAs

template <int NRB>
struct SShape {
  static constexpr int kRows = NRB * 16;
  static constexpr int kSlots = kRows * (kPBK / 8);
  static constexpr int kNS = (kSlots + kSThreads - 1) / kSThreads;           // slots per thread
  static constexpr int kFullWaves = (kSlots - (kNS - 1) * kSThreads) / kWave;  // waves with kNS
  static_assert(kFullWaves * kWave == kSlots - (kNS - 1) * kSThreads && kFullWaves >= 1,
                "the last slot set must cover whole waves");
};

template <typename T, int NRB, int NS>
__device__ __forceinline__ void dcn_s_body(const HParams &p, const TapGeo *geo,
                                           T (*As)[NRB * 16 * kPLDA], T *stage, int n0, int nk,
                                           int lane, int wave, int tid, int4v (&br0)[kPKH][2],
                                           int4v (&br1)[kPKH][2]) {
  using V = Vec<T, 8>;
  constexpr int KV = kPBK / 8;
  constexpr int NF = 2 * NRB;        // A fragments per step (k-half x row block)
  constexpr int NP = NS * 8;         // blend pieces per step (slot x element)
  const int TT = p.taps;
  const int spt = p.C / kPBK;        // K steps per tap
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(p.x, p.x_bytes);
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
  const uint32_t xoob = p.x_bytes;
  const int kv = tid % KV;

  // B fragments of the wave's 32 columns (2 blocks of 16); the K step is the scalar offset.
  uint32_t bo[kPKH][2];
#pragma unroll
  for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
      bo[kh][cb] = b_frag_offset(n0 + wave * 32 + cb * 16 + (lane & 15), kh, lane, p.nb_total,
                                 p.kb_total, p.w_bytes);
  auto issue_b = [&](int ks, int4v (&br)[kPKH][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb)
        br[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(
            wr, bo[kh][cb], (uint32_t)ks * (uint32_t)(kPBK / 16) * 1024u, 0);
  };

  // Gather slots.
  uint32_t go[NS][4];   // corner offsets of the slot's current tap (+ k-vector)
  V ra[NS][4];          // the slot's corners of the next step to blend
  auto slot_row = [&](int i) __attribute__((always_inline)) { return (tid + i * kSThreads) / KV; };
  auto issue_slot = [&](int i, int ks) __attribute__((always_inline)) {
    const int t = ks / spt, cs = ks - t * spt;
    if (cs == 0) {
      if (t < TT) {
        const int4v o = *reinterpret_cast<const int4v *>(geo[slot_row(i) * TT + t].o);
#pragma unroll
        for (int q = 0; q < 4; ++q)
          go[i][q] = (uint32_t)o[q] == xoob ? xoob : (uint32_t)o[q] + (uint32_t)(kv * 8 * sizeof(T));
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q) go[i][q] = xoob;
      }
    }
    const uint32_t so = (uint32_t)(cs * kPBK * sizeof(T));
#pragma unroll
    for (int q = 0; q < 4; ++q)
      ra[i][q] = __builtin_bit_cast(V, __builtin_amdgcn_raw_buffer_load_b128(xr, go[i][q], so, 0));
  };

  floatx4 acc[NRB][2];
#pragma unroll
  for (int i = 0; i < NRB; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Step ks: the MFMAs of A buffer ks % 2 (fragment f = kh * NRB + rb read kSAhead
  // fragments before its MFMAs), with the blend of step ks + 1 into the other buffer
  // spread over the fragments: piece p (slot p / 8, element p % 8: four fused
  // multiply-adds in fp32) goes with fragment p * NF / NP; after a slot's eighth element
  // its A-tile store and its loads of step ks + 2. The order is fixed with sched_barriers
  // (and each element's sum is pinned where it is computed), so the vector ALU work issues
  // between the matrix-core instructions. Then B(ks + 2) and the barrier.
  auto step = [&](int ks, int4v (&br)[kPKH][2]) __attribute__((always_inline)) {
    const T *tile = &As[ks & 1][0];
    T *next = &As[(ks + 1) & 1][0];
    const int tb = min((ks + 1) / spt, TT - 1);  // tap of the step being blended (clamped)
    int4v af[NF];
    auto read_frag = [&](int f) __attribute__((always_inline)) {
      af[f] = *reinterpret_cast<const int4v *>(
          &tile[a_off((f % NRB) * 16 + (lane & 15), (f / NRB) * 4 + (lane >> 4))]);
    };
    float4 w4[NS];
#pragma unroll
    for (int i = 0; i < NS; ++i)
      w4[i] = *reinterpret_cast<const float4 *>(geo[slot_row(i) * TT + tb].w);
#pragma unroll
    for (int f = 0; f < kSAhead; ++f) read_frag(f);
    float bl[8];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
      if (f + kSAhead < NF) read_frag(f + kSAhead);
      const int kh = f / NRB, rbi = f % NRB;
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) acc[rbi][cb] = mfma16x16<T>(af[f], br[kh][cb], acc[rbi][cb]);
#pragma unroll
      for (int pc = 0; pc < NP; ++pc) {
        if (pc * NF / NP != f) continue;
        const int i = pc / 8, e = pc % 8;
        float sum = __builtin_fmaf(w4[i].x, (float)ra[i][0].v[e], 0.f);
        sum = __builtin_fmaf(w4[i].y, (float)ra[i][1].v[e], sum);
        sum = __builtin_fmaf(w4[i].z, (float)ra[i][2].v[e], sum);
        bl[e] = __builtin_fmaf(w4[i].w, (float)ra[i][3].v[e], sum);
        asm volatile("" : "+v"(bl[e]));  // computed here, not moved to its use
        if (e == 7) {
          V o;
#pragma unroll
          for (int u = 0; u < 8; ++u) o.v[u] = static_cast<T>(bl[u]);
          store_vec<T, 8>(&next[a_off(slot_row(i), kv)], o);
          issue_slot(i, ks + 2);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    issue_b(ks + 2, br);
    __syncthreads();
  };

  // prologue: A(0) blended here; the loads of step 1 issued
#pragma unroll
  for (int i = 0; i < NS; ++i) issue_slot(i, 0);
#pragma unroll
  for (int i = 0; i < NS; ++i) {
    const float4 w = *reinterpret_cast<const float4 *>(geo[slot_row(i) * TT].w);
    store_vec<T, 8>(&As[0][a_off(slot_row(i), kv)], blend4<T>(ra[i], w.x, w.y, w.z, w.w));
    issue_slot(i, 1);
  }
  __syncthreads();
  int ks = 0;
  for (; ks + 2 <= nk; ks += 2) {
    step(ks, br0);
    step(ks + 1, br1);
  }
  if (ks < nk) step(ks, br0);

  // Epilogue: lane holds column 32 wave + 16 cb + (lane & 15), rows 4 (lane >> 4) + e.
  const T *bias = static_cast<const T *>(p.bias);
#pragma unroll
  for (int cb = 0; cb < 2; ++cb) {
    const int c = wave * 32 + cb * 16 + (lane & 15);
    const float bv = (bias != nullptr && n0 + c < p.Cout) ? (float)bias[n0 + c] : 0.f;
#pragma unroll
    for (int rbi = 0; rbi < NRB; ++rbi)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = acc[rbi][cb][e] + bv;
        if (p.relu) v = v < 0.f ? 0.f : v;  // NaN stays NaN, as torch.relu
        stage[(rbi * 16 + 4 * (lane >> 4) + e) * kPStage + c] = static_cast<T>(v);
      }
  }
}

// MEGA: the one-launch forward, as dcn_fused_p_kernel's: pass 1 (the offset conv of the
// workgroup's rows, fp32 y with its bias in LDS and, when given, in p.y_out) runs with the
// producer / consumer roles of dcn_fused_p_kernel, pass 2 with the symmetric body.
template <typename T, int GEO, int NRB, bool MEGA>
__global__ void __launch_bounds__(kSThreads) dcn_fused_s_kernel(const PParams pp) {
  using SH = SShape<NRB>;
  using PSH = PShape<NRB>;
  constexpr int kRows = SH::kRows;
  const HParams &p = pp.h;
  __shared__ __attribute__((aligned(16))) TapGeo geo[kRows * kMaxTaps];
  __shared__ __attribute__((aligned(16))) T As[2][kRows * kPLDA];
  __shared__ __attribute__((aligned(16))) T stage[kRows * kPStage];  // the output tile
  static_assert(!MEGA || sizeof(As) >= sizeof(float) * kRows * 3 * kMaxTaps,
                "the offset-conv output must fit in the A ring");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bpx = (int)(gridDim.x >> 3);  // workgroups per XCD (as dcn_fused_p_kernel)
  const int xcd = (int)(blockIdx.x & 7);
  const int xph = 8 / pp.halves;
  const int half = xcd / xph;
  const int nch = (int)gridDim.x / pp.halves;  // row chunks per half
  const int j = (xcd - half * xph) * bpx + (int)(blockIdx.x >> 3);
  const int n0 = half * kPCols;
  const int TT = p.taps;
  const uint32_t xoob = p.x_bytes;
  const int nk = TT * (p.C / kPBK);
  float *ys = reinterpret_cast<float *>(&As[0][0]);
  const int rb0 = (int)((int64_t)pp.rb_total * j / nch);
  const int nrb = (int)((int64_t)pp.rb_total * (j + 1) / nch) - rb0;  // at most NRB
  if (nrb <= 0) return;
  const int m0 = rb0 * 16;
  const int nrows = nrb * 16;

  if constexpr (MEGA) {
    for (int g = tid; g < kRows * TT; g += kSThreads) {
      const int row = g / TT, t = g - row * TT, m = m0 + row;
      geo[g] = (row < nrows && m < p.M) ? tap_geo<T, kGeoRegular>(p, nullptr, 0, m, t)
                                        : empty_geo(xoob);
    }
    __syncthreads();
    if (wave < 4)
      dcn_p_offset_consumer<T, NRB>(p, As, ys, m0, nrb, nk, lane, wave);
    else if (wave - 4 < PSH::kLastWaves)
      dcn_p_producer<T, PSH::kSPT, NRB, true, 2>(p, geo, As, nk, tid - kPProd);
    else
      dcn_p_producer<T, PSH::kSPT - 1, NRB, true, 2>(p, geo, As, nk, tid - kPProd);
    __syncthreads();  // y of every row in ys
  }
  // B fragments of the first two K steps (br0 / br1 of dcn_s_body), issued before the
  // geometry table, which they do not need: their latency runs under it (res4 fp16 61.6 ->
  // 60.8 us, bf16 64.8 -> 64.1 us; dcn_fused_p_kernel loads its first B set the same way)
  int4v br0[kPKH][2], br1[kPKH][2];
  {
    const __amdgpu_buffer_rsrc_t wr = make_rsrc(p.w, p.w_bytes);
#pragma unroll
    for (int kh = 0; kh < kPKH; ++kh)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        const uint32_t bo = b_frag_offset(n0 + wave * 32 + cb * 16 + (lane & 15), kh, lane,
                                          p.nb_total, p.kb_total, p.w_bytes);
        br0[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(wr, bo, 0u, 0);
        br1[kh][cb] = __builtin_amdgcn_raw_buffer_load_b128(wr, bo, (uint32_t)(kPBK / 16) * 1024u, 0);
      }
  }
  for (int g = tid; g < kRows * TT; g += kSThreads) {
    const int row = g / TT, t = g - row * TT, m = m0 + row;
    TapGeo G = empty_geo(xoob);
    if (row < nrows && m < p.M) {
      if constexpr (MEGA)
        G = tap_geo<T, kGeoYF32>(p, ys, row, m, t);   // bias already in ys
      else
        G = tap_geo<T, GEO>(p, p.off, m, m, t);
    }
    geo[g] = G;
  }
  __syncthreads();  // MEGA: ys is dead from here, the A ring is written again
  if (wave < SH::kFullWaves)
    dcn_s_body<T, NRB, SH::kNS>(p, geo, As, stage, n0, nk, lane, wave, tid, br0, br1);
  else
    dcn_s_body<T, NRB, SH::kNS - 1>(p, geo, As, stage, n0, nk, lane, wave, tid, br0, br1);
  __syncthreads();
  T *out = static_cast<T *>(p.out);
  constexpr int kPieces = kPCols / 8;
  for (int i = tid; i < nrows * kPieces; i += kSThreads) {
    const int row = i / kPieces, c = (i - row * kPieces) * 8, m = m0 + row;
    if (m < p.M && n0 + c < p.Cout)
      __builtin_nontemporal_store(*reinterpret_cast<const int4v *>(&stage[row * kPStage + c]),
                                  reinterpret_cast<int4v *>(out + (int64_t)m * p.Cout + n0 + c));
  }
}

template <typename T, int GEO, bool MEGA>
hipError_t launch_s_geo(const PParams &pp, int nrb, hipStream_t stream) {
  const dim3 g(pp.nblocks * pp.rounds), b(kSThreads);
  switch (nrb) {
    case 6: hipLaunchKernelGGL((dcn_fused_s_kernel<T, GEO, 6, MEGA>), g, b, 0, stream, pp); break;
    case 7: hipLaunchKernelGGL((dcn_fused_s_kernel<T, GEO, 7, MEGA>), g, b, 0, stream, pp); break;
    case 8: hipLaunchKernelGGL((dcn_fused_s_kernel<T, GEO, 8, MEGA>), g, b, 0, stream, pp); break;
    case 9: hipLaunchKernelGGL((dcn_fused_s_kernel<T, GEO, 9, MEGA>), g, b, 0, stream, pp); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// The persistent kernels run one workgroup per CU over one 256-column half of Cout. The
// 16-row blocks of M are cut into `rounds` balanced chunks per CU (the grid has rounds
// workgroups per CU, one chunk each), rounds chosen so a chunk has at most 9 blocks, and
// the tile is sized to the largest chunk (NRB blocks,
// so a chunk leaves at most one block of its tile with zero geometry): NRB 6-9 runs the
// symmetric kernel (dcn_fused_s_kernel), NRB 2-5 the producer / consumer kernel
// (dcn_fused_p_kernel). So any M runs on every CU (B = 6 res4: one round of 8-9 blocks;
// res5, two column halves: one round of 4-5 blocks). The CU count is read once per device
// (device_cus).
struct PConfig {
  int nblocks = 0, nrb = 0, halves = 0, rounds = 0;
};
PConfig p_config_for(const HParams &p, int geo) {
  PConfig c;
  if (geo == kGeoRegular || p.C % 64 != 0 || p.Cout <= 128 || p.Cout > 2 * kPCols) return c;
  // the output tile leaves in 16-byte pieces of rows
  if (p.Cout % 8 != 0 || reinterpret_cast<uintptr_t>(p.out) % 16 != 0) return c;
  const int cus = device_cus();
  const int nb = (cus / 8) * 8;
  if (nb < 8) return c;
  const int halves = p.Cout > kPCols ? 2 : 1;
  const int64_t rb = (int64_t)((p.M + 15) / 16);
  const int64_t nbh = nb / halves;
  const int64_t rounds = std::max<int64_t>(1, (rb + nbh * 9 - 1) / (nbh * 9));
  const int64_t per = (rb + nbh * rounds - 1) / (nbh * rounds);  // largest chunk
  if (rounds > (1 << 20)) return c;
  c.nblocks = nb;
  c.nrb = (int)std::max<int64_t>(2, per);
  c.halves = halves;
  c.rounds = (int)rounds;
  return c;
}

template <typename T, int GEO, bool MEGA>
hipError_t launch_p_geo(const PParams &pp, int nrb, hipStream_t stream) {
  const dim3 g(pp.nblocks * pp.rounds), b(kPThreads);
  switch (nrb) {
    case 2: hipLaunchKernelGGL((dcn_fused_p_kernel<T, GEO, 2, MEGA>), g, b, 0, stream, pp); break;
    case 3: hipLaunchKernelGGL((dcn_fused_p_kernel<T, GEO, 3, MEGA>), g, b, 0, stream, pp); break;
    case 4: hipLaunchKernelGGL((dcn_fused_p_kernel<T, GEO, 4, MEGA>), g, b, 0, stream, pp); break;
    case 5: hipLaunchKernelGGL((dcn_fused_p_kernel<T, GEO, 5, MEGA>), g, b, 0, stream, pp); break;
    default: return hipErrorInvalidValue;  // 6-9 blocks run dcn_fused_s_kernel
  }
  return hipGetLastError();
}

template <typename T>
hipError_t launch_p(const HParams &h, int geo, const PConfig &c, bool mega,
                    hipStream_t stream) {
  PParams pp;
  pp.h = h;
  pp.rb_total = (h.M + 15) / 16;
  pp.nblocks = c.nblocks;
  pp.halves = c.halves;
  pp.rounds = c.rounds;
  // 6-9 blocks: the symmetric kernel (the blend arithmetic of 144 rows split over both
  // waves of each SIMD: res4 fp16 69.2 -> 67.3 us, bf16 77.5 -> 71.5 us); up to 5 blocks
  // the producer / consumer kernel (the symmetric one measured res5 fp16 76.4 -> 78.1 us,
  // bf16 78.3 -> 83.4 us: less blend work per SIMD, twice the A-tile reads).
  if (c.nrb >= 6) {
    if (mega) return launch_s_geo<T, kGeoYF32, true>(pp, c.nrb, stream);
    if (geo == kGeoY) return launch_s_geo<T, kGeoY, false>(pp, c.nrb, stream);
    if (geo == kGeoYF32) return launch_s_geo<T, kGeoYF32, false>(pp, c.nrb, stream);
    return launch_s_geo<T, kGeoMask, false>(pp, c.nrb, stream);
  }
  if (mega) return launch_p_geo<T, kGeoYF32, true>(pp, c.nrb, stream);
  if (geo == kGeoY) return launch_p_geo<T, kGeoY, false>(pp, c.nrb, stream);
  if (geo == kGeoYF32) return launch_p_geo<T, kGeoYF32, false>(pp, c.nrb, stream);
  return launch_p_geo<T, kGeoMask, false>(pp, c.nrb, stream);
}

template <typename T>
hipError_t launch_t(const HParams &p, int geo, hipStream_t stream) {
  const PConfig c = p_config_for(p, geo);
  if (c.nblocks) return launch_p<T>(p, geo, c, false, stream);
  return p.C % 64 == 0 ? launch_tt<T, true>(p, geo, stream) : launch_tt<T, false>(p, geo, stream);
}

}  // namespace

int64_t dcn_packed_weight_elems(int dtype, int cout, int K) {
  if (dtype == 0) return (int64_t)cout * K;
  const int64_t nb = (cout + 31) / 32, kb = (K + 15) / 16;
  return nb * kb * 64 * 8;
}

hipError_t launch_dcn_pack_weight(int dtype, const void *weight, int cout, int C, int T,
                                  void *packed, hipStream_t stream, bool src_tc) {
  const int K = C * T;
  if (dtype == 0) {
    const int64_t total = (int64_t)cout * K;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(pack_weight_kc_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, static_cast<const float *>(weight), static_cast<float *>(packed),
                       C, T, total, src_tc);
    return hipGetLastError();
  }
  const int KB = (K + 15) / 16;
  const int64_t chunks = (int64_t)((cout + 31) / 32) * KB * 64;
  if (chunks == 0) return hipSuccess;
  const bool aligned = reinterpret_cast<uintptr_t>(weight) % 16 == 0 &&
                       reinterpret_cast<uintptr_t>(packed) % 16 == 0;
  if (aligned && src_tc && K % 8 == 0) {
    hipLaunchKernelGGL(pack_weight_frag_tc_kernel, dim3((unsigned)((chunks + 255) / 256)),
                       dim3(256), 0, stream, static_cast<const uint16_t *>(weight),
                       static_cast<uint16_t *>(packed), cout, K, KB, chunks);
    return hipGetLastError();
  }
  if (aligned && !src_tc && C % 16 == 0 && T <= kPackMaxT) {
    hipLaunchKernelGGL(pack_weight_frag_lds_kernel, dim3((unsigned)((cout + 31) / 32), C / 16),
                       dim3(256), 0, stream, static_cast<const uint16_t *>(weight),
                       static_cast<uint16_t *>(packed), cout, C, T, KB);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(pack_weight_frag_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256),
                     0, stream, static_cast<const uint16_t *>(weight),
                     static_cast<uint16_t *>(packed), cout, C, T, KB, chunks, src_tc);
  return hipGetLastError();
}

bool dcn_fused_h_supported(const DcnGeom &g) { return g.kernel_h * g.kernel_w <= kMaxTaps; }

namespace {
HParams make_hparams(int dtype, const DcnGeom &g, int channels_out, const void *x,
                     const void *off, const void *msk, const void *w_packed, const void *bias,
                     void *out, const float *y_bias, bool relu) {
  HParams p{};
  p.x = x; p.off = off; p.msk = msk; p.w = w_packed; p.bias = bias; p.out = out;
  p.yb = y_bias; p.relu = relu ? 1 : 0;
  p.C = g.channels; p.H = g.height; p.W = g.width; p.Ho = g.height_col; p.Wo = g.width_col;
  p.Cout = channels_out; p.kh = g.kernel_h; p.kw = g.kernel_w;
  p.ph = g.pad_h; p.pw = g.pad_w; p.sh = g.stride_h; p.sw = g.stride_w;
  p.dh = g.dil_h; p.dw = g.dil_w;
  p.M = g.batch * g.height_col * g.width_col;
  p.taps = g.kernel_h * g.kernel_w;
  p.K = p.taps * g.channels;
  p.nb_total = (channels_out + 31) / 32;
  p.kb_total = (p.K + 15) / 16;
  p.x_bytes = (uint32_t)((int64_t)g.batch * g.height * g.width * g.channels * 2);
  p.w_bytes = (uint32_t)(dcn_packed_weight_elems(dtype, channels_out, p.K) * 2);
  return p;
}
}  // namespace

hipError_t launch_dcn_fused_h(int dtype, const DcnGeom &g, int channels_out, const void *x,
                              const void *off, int geo, const void *msk,
                              const void *w_packed, const void *bias, void *out,
                              hipStream_t stream, const float *y_bias, bool relu) {
  const HParams p =
      make_hparams(dtype, g, channels_out, x, off, msk, w_packed, bias, out, y_bias, relu);
  switch (dtype) {
    case 1: return launch_t<f16>(p, geo, stream);
    case 2: return launch_t<bf16>(p, geo, stream);
    default: return hipErrorInvalidValue;
  }
}

// The one-launch form runs where Cout fits one 256-column half. With two halves every
// workgroup pair would compute the offset conv of the same rows, so the caller runs the
// offset conv once into y (the row-segment kernel) and then the fused kernel reading y:
// res5 fp16 113 -> 88 us, bf16 117 -> 91 us (res4, one half, stays in one launch: 88-90 us
// against 26 + 65 us in two).
bool dcn_mega_supported(int dtype, const DcnGeom &g, int channels_out, const void *out) {
  if ((dtype != 1 && dtype != 2) || g.deformable_group != 1 ||
      g.kernel_h * g.kernel_w > kMaxTaps)
    return false;
  const HParams p = make_hparams(dtype, g, channels_out, nullptr, nullptr, nullptr, nullptr,
                                 nullptr, const_cast<void *>(out), nullptr, false);
  const PConfig c = p_config_for(p, kGeoYF32);
  return c.nblocks != 0 && c.halves == 1;
}

hipError_t launch_dcn_mega(int dtype, const DcnGeom &g, int channels_out, const void *x,
                           const void *w_off_packed, const float *b_off,
                           const void *w_packed, const void *bias, bool relu, float *y_out,
                           void *out, hipStream_t stream) {
  if (!dcn_mega_supported(dtype, g, channels_out, out)) return hipErrorInvalidValue;
  HParams p = make_hparams(dtype, g, channels_out, x, nullptr, nullptr, w_packed, bias, out,
                           nullptr, relu);
  p.w2 = w_off_packed;
  p.b2 = b_off;
  p.y_out = y_out;
  p.w2_bytes = (uint32_t)(dcn_packed_weight_elems(dtype, 3 * p.taps, p.K) * 2);
  const PConfig c = p_config_for(p, kGeoYF32);
  switch (dtype) {
    case 1: return launch_p<f16>(p, kGeoYF32, c, true, stream);
    case 2: return launch_p<bf16>(p, kGeoYF32, c, true, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
