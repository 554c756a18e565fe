// Multi-scale deformable attention, forward, for gfx950.
//
// Semantics (naotic/bev-kernels, ms_deform_attn_kernels.cuh:7-49, :252-259, :281-283):
//   out[b, q, h*D + c] = sum_l sum_p attn[b,q,h,l,p] * bilinear_l(value, loc[b,q,h,l,p])
//   h_im = loc_y * H_l - 0.5, w_im = loc_x * W_l - 0.5; a sample contributes only if
//   -1 < h_im < H_l and -1 < w_im < W_l, and each of its four corners is zero outside
//   the level. value[b, level_start[l] + y*W_l + x, h, c].
//
// Kernels:
//   * msda_wave_kernel / msda_wave_lds_kernel: one wavefront owns UPW (b, q, head)
//     units. G = D/VEC lanes cover the head_dim channels of one sample with 16-byte
//     loads; the other lane groups take other (level, point) samples at the same time
//     and the partial sums meet in a butterfly over the lane groups. All corner loads of
//     a unit are issued before the first use. Corner loads are buffer loads: an invalid
//     corner gets an out-of-range offset and reads 0 without a memory request, so the
//     zero padding is branch-free.
//     The _lds variant (many samples per unit) computes each sample's geometry once,
//     in one lane, with the attention weight folded into the four corner weights, and
//     shares it with the sample's lane group through LDS; the plain variant (few
//     samples, or L/P known only at run time) lets every lane of the group compute it.
//   * Work order: units are enumerated per (batch, head-group) slice, queries in order,
//     slices one after the other. All 8 XCDs then work on the same slice at the same
//     time: each XCD's L2 holds one slice (3.95 MB for fp32 SCA) and a line one XCD
//     pulls from HBM is a MALL hit for the others.
//   * msda_generic_kernel: one thread per output element, any shape and dtype.
#include "bevk_common.h"
#include "bevk_launch.h"

namespace bevk {
namespace {

constexpr int kBlock = 256;            // 4 waves
constexpr int kWavesPerBlock = kBlock / kWave;

template <typename T> __device__ __forceinline__ void load_loc(const T *p, float &x, float &y) {
  x = static_cast<float>(load_nt(p));
  y = static_cast<float>(load_nt(p + 1));
}
template <> __device__ __forceinline__ void load_loc<float>(const float *p, float &x, float &y) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = __builtin_nontemporal_load(reinterpret_cast<const f2 *>(p));
  x = v.x;
  y = v.y;
}

struct WaveParams {
  const void *value;
  const int64_t *shapes;
  const int64_t *lsi;
  const void *loc;
  const void *attn;
  void *out;
  int S, NH, NQ, nl, np;
  int heads_per_slice;    // heads sharing one slice (2 when two heads fill a 128 B line)
  int slices_per_batch;   // NH / heads_per_slice
  int blocks_per_slice;   // ceil(NQ * heads_per_slice / units_per_block)
  uint32_t batch_bytes;   // bytes of value per batch (buffer range; < 2^31)
};

// NL/NP > 0: compile-time level/point counts; 0: read from params.
template <typename T, int D, int VEC, int NL, int NP, int UPW>
__global__ void __launch_bounds__(kBlock) msda_wave_kernel(const WaveParams p) {
  using V = Vec<T, VEC>;
  constexpr int G = D / VEC;           // lanes per sample
  constexpr int LPU = kWave / UPW;     // lanes per unit
  constexpr int SPU = LPU / G;         // samples in flight per unit
  static_assert(G >= 1 && G <= kWave && (kWave % (G * UPW)) == 0, "bad lane split");
  constexpr bool kStatic = NL > 0 && NP > 0;
  const int nl = kStatic ? NL : p.nl;
  const int np = kStatic ? NP : p.np;
  const int ns = nl * np;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;

  // block -> (slice, chunk): slices one after the other, queries in order.
  const int slice = blockIdx.x / p.blocks_per_slice;
  const int chunk = blockIdx.x - slice * p.blocks_per_slice;
  const int b = slice / p.slices_per_batch;
  const int hg = slice - b * p.slices_per_batch;
  const int local = (chunk * kWavesPerBlock + wave) * UPW + lane / LPU;
  const int q = local / p.heads_per_slice;
  const int h = hg * p.heads_per_slice + (local - q * p.heads_per_slice);
  const bool active = q < p.NQ;
  const int qc = active ? q : p.NQ - 1;
  const int64_t unit = ((int64_t)b * p.NQ + qc) * p.NH + h;

  const int ul = lane & (LPU - 1);
  const int g = ul / G;
  const int c0 = (ul - g * G) * VEC;

  const T *vbase = static_cast<const T *>(p.value) + (int64_t)b * p.S * p.NH * D;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(vbase, p.batch_bytes);
  const uint32_t kOOB = p.batch_bytes;  // any load at this offset is out of range -> 0
  const int pos_stride = p.NH * D;       // elements between neighbouring positions
  const int head_off = h * D + c0;

  const T *locp = static_cast<const T *>(p.loc) + unit * ns * 2;
  const T *attp = static_cast<const T *>(p.attn) + unit * ns;

  // Level table: compile-time NL keeps it in (scalar) registers.
  constexpr int NLR = NL > 0 ? NL : 1;
  int lvH[NLR], lvW[NLR], lvS[NLR];
  if constexpr (NL > 0) {
#pragma unroll
    for (int l = 0; l < NL; ++l) {
      lvH[l] = (int)p.shapes[2 * l];
      lvW[l] = (int)p.shapes[2 * l + 1];
      lvS[l] = (int)p.lsi[l];
    }
  }

  float acc[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = 0.f;

  auto sample = [&](int s, float &wgt, float &w1, float &w2, float &w3, float &w4,
                    uint32_t &o1, uint32_t &o2, uint32_t &o3, uint32_t &o4) {
    int l, Hl, Wl, Sl;
    if constexpr (NL > 0) {
      l = s / NP;
      Hl = lvH[0];
      Wl = lvW[0];
      Sl = lvS[0];
#pragma unroll
      for (int i = 1; i < NL; ++i)
        if (l == i) { Hl = lvH[i]; Wl = lvW[i]; Sl = lvS[i]; }
    } else {
      l = s / np;
      Hl = (int)p.shapes[2 * l];
      Wl = (int)p.shapes[2 * l + 1];
      Sl = (int)p.lsi[l];
    }
    float x, y;
    load_loc<T>(locp + 2 * s, x, y);
    wgt = static_cast<float>(load_nt(attp + s));
    const float him = y * (float)Hl - 0.5f;
    const float wim = x * (float)Wl - 0.5f;
    o1 = o2 = o3 = o4 = kOOB;
    w1 = w2 = w3 = w4 = 0.f;
    const bool in = active && him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl;
    if (!in) wgt = 0.f;
    if (in) {
      const float fh = floorf(him), fw = floorf(wim);
      const int hl = (int)fh, wl = (int)fw;
      const float lh = him - fh, lw = wim - fw;
      const float hh = 1.f - lh, hw = 1.f - lw;
      w1 = hh * hw; w2 = hh * lw; w3 = lh * hw; w4 = lh * lw;
      const int r0 = Sl + hl * Wl + wl;  // position of the (hl, wl) corner
      const uint32_t base = (uint32_t)(r0 * pos_stride + head_off) * sizeof(T);
      const uint32_t dx = (uint32_t)(pos_stride * sizeof(T));
      const uint32_t dy = (uint32_t)(Wl * pos_stride * sizeof(T));
      const bool y0 = hl >= 0, y1 = hl + 1 <= Hl - 1;
      const bool x0 = wl >= 0, x1 = wl + 1 <= Wl - 1;
      if (y0 && x0) o1 = base;
      if (y0 && x1) o2 = base + dx;
      if (y1 && x0) o3 = base + dy;
      if (y1 && x1) o4 = base + dy + dx;
    }
  };

  auto combine = [&](float wgt, float w1, float w2, float w3, float w4, const V &v1,
                     const V &v2, const V &v3, const V &v4) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) {
      const float bil = w1 * (float)v1.v[k] + w2 * (float)v2.v[k] + w3 * (float)v3.v[k] +
                        w4 * (float)v4.v[k];
      acc[k] += bil * wgt;
    }
  };

  if constexpr (kStatic) {
    // Issue every corner load of the unit before the first use.
    constexpr int NITER = (NL * NP + SPU - 1) / SPU;
    float wgt[NITER], w1[NITER], w2[NITER], w3[NITER], w4[NITER];
    V v1[NITER], v2[NITER], v3[NITER], v4[NITER];
#pragma unroll
    for (int it = 0; it < NITER; ++it) {
      const int s = it * SPU + g;
      uint32_t o1, o2, o3, o4;
      if ((NL * NP) % SPU == 0 || s < NL * NP) {
        sample(s, wgt[it], w1[it], w2[it], w3[it], w4[it], o1, o2, o3, o4);
      } else {
        wgt[it] = w1[it] = w2[it] = w3[it] = w4[it] = 0.f;
        o1 = o2 = o3 = o4 = kOOB;
      }
      v1[it] = buffer_load_vec<T, VEC>(rsrc, o1);
      v2[it] = buffer_load_vec<T, VEC>(rsrc, o2);
      v3[it] = buffer_load_vec<T, VEC>(rsrc, o3);
      v4[it] = buffer_load_vec<T, VEC>(rsrc, o4);
    }
#pragma unroll
    for (int it = 0; it < NITER; ++it)
      combine(wgt[it], w1[it], w2[it], w3[it], w4[it], v1[it], v2[it], v3[it], v4[it]);
  } else {
    for (int s = g; s < ns; s += SPU) {
      float wgt, w1, w2, w3, w4;
      uint32_t o1, o2, o3, o4;
      sample(s, wgt, w1, w2, w3, w4, o1, o2, o3, o4);
      const V v1 = buffer_load_vec<T, VEC>(rsrc, o1);
      const V v2 = buffer_load_vec<T, VEC>(rsrc, o2);
      const V v3 = buffer_load_vec<T, VEC>(rsrc, o3);
      const V v4 = buffer_load_vec<T, VEC>(rsrc, o4);
      combine(wgt, w1, w2, w3, w4, v1, v2, v3, v4);
    }
  }

  // Sum the lane groups of one unit (lanes that share a channel slice).
#pragma unroll
  for (int m = G; m < LPU; m <<= 1) {
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] += __shfl_xor(acc[k], m);
  }

  if (active && g == 0) {
    V o;
#pragma unroll
    for (int k = 0; k < VEC; ++k) o.v[k] = from_acc<T>(acc[k]);
    store_vec_nt<T, VEC>(static_cast<T *>(p.out) + unit * D + c0, o);
  }
}

// Geometry of one sample, shared through LDS: corner weights (bilinear x attention,
// zero for invalid corners) and corner byte offsets (out-of-range sentinel if invalid).
struct SampleGeo {
  float w[4];
  uint32_t o[4];
};

// Compile-time L/P with UPW * L * P <= 64: lane i of the wave computes sample i of the
// wave's UPW units, then every lane group gathers its samples' corners.
template <typename T, int D, int VEC, int NL, int NP, int UPW>
__global__ void __launch_bounds__(kBlock) msda_wave_lds_kernel(const WaveParams p) {
  using V = Vec<T, VEC>;
  constexpr int G = D / VEC, LPU = kWave / UPW, SPU = LPU / G, NS = NL * NP;
  constexpr int NITER = (NS + SPU - 1) / SPU;
  static_assert(UPW * NS <= kWave && G >= 1 && (kWave % (G * UPW)) == 0, "bad lane split");
  __shared__ SampleGeo geo[kWavesPerBlock][UPW * NS];

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int slice = blockIdx.x / p.blocks_per_slice;
  const int chunk = blockIdx.x - slice * p.blocks_per_slice;
  const int b = slice / p.slices_per_batch;
  const int hg = slice - b * p.slices_per_batch;
  const int pos_stride = p.NH * D;
  const uint32_t kOOB = p.batch_bytes;

  // Phase 1: one lane per (unit, sample).
  if (lane < UPW * NS) {
    const int u = lane / NS, s = lane - (lane / NS) * NS;
    const int local = (chunk * kWavesPerBlock + wave) * UPW + u;
    const int q = local / p.heads_per_slice;
    const int h = hg * p.heads_per_slice + (local - q * p.heads_per_slice);
    const bool active = q < p.NQ;
    const int qc = active ? q : p.NQ - 1;
    const int64_t unit = ((int64_t)b * p.NQ + qc) * p.NH + h;
    const int l = s / NP;
    const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1], Sl = (int)p.lsi[l];
    float x, y;
    load_loc<T>(static_cast<const T *>(p.loc) + (unit * NS + s) * 2, x, y);
    const float a = static_cast<float>(load_nt(static_cast<const T *>(p.attn) + unit * NS + s));
    const float him = y * (float)Hl - 0.5f, wim = x * (float)Wl - 0.5f;
    SampleGeo sg;
    sg.w[0] = sg.w[1] = sg.w[2] = sg.w[3] = 0.f;
    sg.o[0] = sg.o[1] = sg.o[2] = sg.o[3] = kOOB;
    if (active && him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl) {
      const float fh = floorf(him), fw = floorf(wim);
      const int hl = (int)fh, wl = (int)fw;
      const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
      const uint32_t es = (uint32_t)sizeof(T);
      const uint32_t base = (uint32_t)((Sl + hl * Wl + wl) * pos_stride + h * D) * es;
      const uint32_t dx = (uint32_t)pos_stride * es, dy = (uint32_t)(Wl * pos_stride) * es;
      const bool y0 = hl >= 0, y1 = hl + 1 <= Hl - 1, x0 = wl >= 0, x1 = wl + 1 <= Wl - 1;
      if (y0 && x0) { sg.w[0] = hh * hw * a; sg.o[0] = base; }
      if (y0 && x1) { sg.w[1] = hh * lw * a; sg.o[1] = base + dx; }
      if (y1 && x0) { sg.w[2] = lh * hw * a; sg.o[2] = base + dy; }
      if (y1 && x1) { sg.w[3] = lh * lw * a; sg.o[3] = base + dy + dx; }
    }
    geo[wave][lane] = sg;
  }
  // The wave reads what its own lanes wrote: order the LDS accesses within the wave.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

  // Phase 2: lane group gi of unit u gathers samples gi, gi + SPU, ...
  const int u = lane / LPU, ul = lane & (LPU - 1), gi = ul / G, c0 = (ul - gi * G) * VEC;
  const int local = (chunk * kWavesPerBlock + wave) * UPW + u;
  const int q = local / p.heads_per_slice;
  const int h = hg * p.heads_per_slice + (local - q * p.heads_per_slice);
  const T *vbase = static_cast<const T *>(p.value) + (int64_t)b * p.S * p.NH * D;
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(vbase, p.batch_bytes);
  const uint32_t cb = (uint32_t)(c0 * sizeof(T));
  V v[NITER][4];
  float w[NITER][4];
#pragma unroll
  for (int it = 0; it < NITER; ++it) {
    const int s = it * SPU + gi;
    if (NS % SPU == 0 || s < NS) {
      const SampleGeo sg = geo[wave][u * NS + s];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        w[it][c] = sg.w[c];
        v[it][c] = buffer_load_vec<T, VEC>(rsrc, sg.o[c] == kOOB ? kOOB : sg.o[c] + cb);
      }
    } else {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        w[it][c] = 0.f;
        v[it][c] = buffer_load_vec<T, VEC>(rsrc, kOOB);
      }
    }
  }
  float acc[VEC];
#pragma unroll
  for (int k = 0; k < VEC; ++k) acc[k] = 0.f;
#pragma unroll
  for (int it = 0; it < NITER; ++it)
#pragma unroll
    for (int k = 0; k < VEC; ++k)
      acc[k] += w[it][0] * (float)v[it][0].v[k] + w[it][1] * (float)v[it][1].v[k] +
                w[it][2] * (float)v[it][2].v[k] + w[it][3] * (float)v[it][3].v[k];
#pragma unroll
  for (int m = G; m < LPU; m <<= 1)
#pragma unroll
    for (int k = 0; k < VEC; ++k) acc[k] += __shfl_xor(acc[k], m);
  if (q < p.NQ && gi == 0) {
    V o;
#pragma unroll
    for (int k = 0; k < VEC; ++k) o.v[k] = from_acc<T>(acc[k]);
    const int64_t unit = ((int64_t)b * p.NQ + q) * p.NH + h;
    store_vec_nt<T, VEC>(static_cast<T *>(p.out) + unit * D + c0, o);
  }
}

// One thread per output element (b, q, h, c); any heads / channels / levels / points.
template <typename T>
__global__ void __launch_bounds__(kBlock) msda_generic_kernel(
    const T *__restrict__ value, const int64_t *__restrict__ shapes,
    const int64_t *__restrict__ lsi, const T *__restrict__ loc, const T *__restrict__ attn,
    T *__restrict__ out, int S, int NH, int D, int NL, int NQ, int NP, int64_t n) {
  using A = typename Acc<T>::type;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += stride) {
    const int c = (int)(idx % D);
    const int64_t unit = idx / D;  // ((b * NQ + q) * NH + h)
    const int h = (int)(unit % NH);
    const int64_t b = unit / ((int64_t)NH * NQ);
    const int64_t pos_stride = (int64_t)NH * D;
    const T *vb = value + b * S * pos_stride + (int64_t)h * D + c;
    const T *lp = loc + unit * NL * NP * 2;
    const T *ap = attn + unit * NL * NP;
    A acc = 0;
    for (int l = 0; l < NL; ++l) {
      const int Hl = (int)shapes[2 * l];
      const int Wl = (int)shapes[2 * l + 1];
      const T *vl = vb + lsi[l] * pos_stride;
      for (int pt = 0; pt < NP; ++pt, lp += 2, ++ap) {
        const A x = static_cast<A>(lp[0]);
        const A y = static_cast<A>(lp[1]);
        const A w = static_cast<A>(ap[0]);
        const A him = y * (A)Hl - (A)0.5;
        const A wim = x * (A)Wl - (A)0.5;
        if (him > (A)-1 && wim > (A)-1 && him < (A)Hl && wim < (A)Wl) {
          const A fh = floor(him), fw = floor(wim);
          const int hl = (int)fh, wl = (int)fw;
          const A lh = him - fh, lw = wim - fw;
          const A hh = (A)1 - lh, hw = (A)1 - lw;
          A v1 = 0, v2 = 0, v3 = 0, v4 = 0;
          const int64_t r0 = (int64_t)hl * Wl + wl;
          // Positions outside [0, S) (inconsistent level metadata) read as zero.
          const int64_t lo = -lsi[l], hi = (int64_t)S - lsi[l];
          auto in_s = [&](int64_t r) { return r >= lo && r < hi; };
          if (hl >= 0 && wl >= 0 && in_s(r0)) v1 = static_cast<A>(vl[r0 * pos_stride]);
          if (hl >= 0 && wl + 1 <= Wl - 1 && in_s(r0 + 1))
            v2 = static_cast<A>(vl[(r0 + 1) * pos_stride]);
          if (hl + 1 <= Hl - 1 && wl >= 0 && in_s(r0 + Wl))
            v3 = static_cast<A>(vl[(r0 + Wl) * pos_stride]);
          if (hl + 1 <= Hl - 1 && wl + 1 <= Wl - 1 && in_s(r0 + Wl + 1))
            v4 = static_cast<A>(vl[(r0 + Wl + 1) * pos_stride]);
          acc += (hh * hw * v1 + hh * lw * v2 + lh * hw * v3 + lh * lw * v4) * w;
        }
      }
    }
    out[idx] = static_cast<T>(acc);
  }
}

template <typename T>
hipError_t launch_generic(const MsdaArgs &a, hipStream_t stream) {
  const int64_t n = (int64_t)a.batch * a.num_query * a.num_heads * a.channels;
  if (n == 0) return hipSuccess;
  const int64_t want = (n + kBlock - 1) / kBlock;
  const int blocks = (int)(want < (1 << 20) ? want : (1 << 20));
  hipLaunchKernelGGL(msda_generic_kernel<T>, dim3(blocks), dim3(kBlock), 0, stream,
                     static_cast<const T *>(a.value), a.spatial_shapes, a.level_start_index,
                     static_cast<const T *>(a.sampling_loc),
                     static_cast<const T *>(a.attn_weight), static_cast<T *>(a.output),
                     a.spatial_size, a.num_heads, a.channels, a.num_levels, a.num_query,
                     a.num_point, n);
  return hipGetLastError();
}

constexpr int upw_for(int G, int ns) {
  int upw = 1;
  while (upw * 2 * G * ns <= kWave && (kWave % (upw * 2 * G)) == 0) upw *= 2;
  return upw;
}

template <typename T, int D, int NL, int NP>
hipError_t launch_wave_t(const MsdaArgs &a, hipStream_t stream) {
  constexpr int VEC = 16 / sizeof(T) < D ? 16 / sizeof(T) : D;
  constexpr int G = D / VEC;
  constexpr bool kStatic = NL > 0 && NP > 0;
  // Many samples per unit: shared geometry through LDS, two units per wave when their
  // samples fit one geometry pass. Few samples: per-lane geometry, units packed so the
  // wave's lanes are all busy.
  constexpr bool kLds = kStatic && NL * NP >= 16 && NL * NP <= kWave;
  constexpr int UPW = kLds ? (2 * NL * NP <= kWave && kWave % (2 * G) == 0 ? 2 : 1)
                           : (kStatic ? upw_for(G, NL * NP) : 1);
  WaveParams p;
  p.value = a.value;
  p.shapes = a.spatial_shapes;
  p.lsi = a.level_start_index;
  p.loc = a.sampling_loc;
  p.attn = a.attn_weight;
  p.out = a.output;
  p.S = a.spatial_size;
  p.NH = a.num_heads;
  p.NQ = a.num_query;
  p.nl = a.num_levels;
  p.np = a.num_point;
  // Two heads share one 128 B line when D * sizeof(T) == 64: keep them together.
  int hps = 1;
  while (hps * 2 <= a.num_heads && (a.num_heads % (hps * 2)) == 0 &&
         hps * 2 * D * (int)sizeof(T) <= 128)
    hps *= 2;
  p.heads_per_slice = hps;
  p.slices_per_batch = a.num_heads / hps;
  const int units_per_block = kWavesPerBlock * UPW;
  const int64_t units_per_slice = (int64_t)a.num_query * hps;
  p.blocks_per_slice = (int)((units_per_slice + units_per_block - 1) / units_per_block);
  const int64_t slices = (int64_t)a.batch * p.slices_per_batch;
  p.batch_bytes = (uint32_t)((int64_t)a.spatial_size * a.num_heads * D * sizeof(T));
  const int64_t blocks = slices * p.blocks_per_slice;
  if (blocks == 0) return hipSuccess;
  if constexpr (kLds)
    hipLaunchKernelGGL((msda_wave_lds_kernel<T, D, VEC, NL, NP, UPW>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, stream, p);
  else
    hipLaunchKernelGGL((msda_wave_kernel<T, D, VEC, NL, NP, UPW>), dim3((unsigned)blocks),
                       dim3(kBlock), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_wave(const MsdaArgs &a, hipStream_t stream) {
  const int L = a.num_levels, P = a.num_point;
  switch (a.channels) {
    case 32:
      if (L == 4 && P == 8) return launch_wave_t<T, 32, 4, 8>(a, stream);  // BEVFormer SCA
      if (L == 1 && P == 4) return launch_wave_t<T, 32, 1, 4>(a, stream);  // BEVFormer TSA
      if (L == 4 && P == 4) return launch_wave_t<T, 32, 4, 4>(a, stream);  // Deformable DETR
      return launch_wave_t<T, 32, 0, 0>(a, stream);
    case 16: return launch_wave_t<T, 16, 0, 0>(a, stream);
    case 64: return launch_wave_t<T, 64, 0, 0>(a, stream);
    case 128: return launch_wave_t<T, 128, 0, 0>(a, stream);
    default: return launch_generic<T>(a, stream);
  }
}

bool wave_supported(int dtype_bytes, const MsdaArgs &a) {
  const int c = a.channels;
  if (!(c == 16 || c == 32 || c == 64 || c == 128)) return false;
  // 32-bit buffer offsets per batch, with room for the out-of-range sentinel.
  const int64_t batch_bytes = (int64_t)a.spatial_size * a.num_heads * c * dtype_bytes;
  if (batch_bytes >= ((int64_t)1 << 31) - 256) return false;
  if ((int64_t)a.num_query * a.num_heads >= ((int64_t)1 << 30)) return false;
  return true;
}

}  // namespace

hipError_t launch_msda_forward(int dtype, const MsdaArgs &a, bool force_generic,
                               hipStream_t stream) {
  switch (dtype) {
    case 0:  // f32
      if (!force_generic && wave_supported(4, a)) return launch_wave<float>(a, stream);
      return launch_generic<float>(a, stream);
    case 1:  // f16
      if (!force_generic && wave_supported(2, a)) return launch_wave<f16>(a, stream);
      return launch_generic<f16>(a, stream);
    case 2:  // bf16
      if (!force_generic && wave_supported(2, a)) return launch_wave<bf16>(a, stream);
      return launch_generic<bf16>(a, stream);
    case 3:  // f64
      return launch_generic<double>(a, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace bevk
