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
//     and the partial sums meet in a butterfly over the lane groups (lane_group_sum). All
//     corner loads of a unit are issued before the first use. Corner loads are buffer
//     loads: an invalid corner gets an out-of-range offset and reads 0 without a memory
//     request, so the zero padding is branch-free.
//     The _lds variant (many samples per unit) computes each sample's geometry once,
//     in one lane, with the attention weight folded into the four corner weights, and
//     shares it with the sample's lane group through LDS; the plain variant (few
//     samples, or L/P known only at run time) lets every lane of the group compute it.
//   * Work order: units are enumerated per (batch, head-group) slice, queries in order,
//     slices one after the other. The _lds variant lets XCD x take the x-th contiguous
//     eighth of that order: each XCD works through its own slices (a whole slice at a
//     time when there are at least 8), so its L2 holds one slice (3.95 MB for fp32 SCA)
//     and every value line is pulled into one L2 only. The plain variant keeps all XCDs
//     on one slice, each on an eighth of its queries (see xcd_chunk).
//   * msda_generic_kernel: one thread per output element, any shape and dtype.
#include <atomic>
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

// Each x[k] summed over lanes i ^ m for m = G, 2G, ..., LPL / 2 (G, LPL powers of two;
// lanes in aligned groups of LPL), i.e. over the lanes of i's group that share i % G; one
// step at a time over all N values. Groups of 32 or more lanes sum on the vector ALU: row
// rotations by 8, 4, ... G inside each 16-lane row (after them a lane holds the sum over
// i + kG mod 16), then the gfx950 row swap (lanes i, i ^ 16) and half-wave swap (i, i ^ 32);
// the swaps return both lanes' values, and their sum is the same in both lanes (against
// LDS-pipe permutes: SCA fp16 242.5 -> 239.0 us, bf16 253.2 -> 250.8 us). Smaller
// groups use LDS-pipe permutes: the rotations took the 16-bit four-point cached kernel
// (16-lane groups) from 151 to 168 registers with spills (DETR fp16 89 -> 93 us).
// Call with every lane of the wave active: the rotations and swaps read other lanes'
// registers (all call sites are outside divergent code).
template <int M> __device__ __forceinline__ float row_ror(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 | M, 0xf, 0xf, false));
}
__device__ __forceinline__ float swap16_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
__device__ __forceinline__ float swap32_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}
template <int G, int LPL, int N> __device__ __forceinline__ void lane_group_sum(float (&x)[N]) {
  static_assert((G & (G - 1)) == 0 && (LPL & (LPL - 1)) == 0 && LPL <= kWave, "lane groups");
  if constexpr (LPL < 32) {
#pragma unroll
    for (int m = G; m < LPL; m <<= 1)
#pragma unroll
      for (int k = 0; k < N; ++k) x[k] += __shfl_xor(x[k], m);
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 8) x[k] += row_ror<8>(x[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 4) x[k] += row_ror<4>(x[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 2) x[k] += row_ror<2>(x[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 1) x[k] += row_ror<1>(x[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 16 && LPL >= 32) x[k] = swap16_sum(x[k]);
#pragma unroll
    for (int k = 0; k < N; ++k) if constexpr (G <= 32 && LPL >= 64) x[k] = swap32_sum(x[k]);
  }
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
  int blocks_per_slice;   // ceil(NQ * heads_per_slice / units_per_block), a multiple of 8
                          // (so the grid is a multiple of 8 blocks)
  uint32_t batch_bytes;   // bytes of value per batch (buffer range; < 2^31)
};

// Two block orders, both running block i on XCD i % 8 (blocks_per_slice and the grid are
// multiples of 8):
// * xcd_chunk (msda_wave_kernel): block r of a slice takes chunk (r % 8) * (bps / 8) + r / 8,
//   so all XCDs work on the same slice, XCD x on one contiguous eighth of its queries.
//   Where sampling locations follow the queries (temporal self-attention over a BEV
//   grid), the value rows an XCD needs stay in its own L2 instead of every XCD fetching
//   every row.
// * xcd_block (msda_wave_lds_kernel): block i takes logical block (i % 8) * (grid / 8) +
//   i / 8 of the slice-major order, so each XCD works through its own slices and every
//   value line of a slice is pulled into one L2 only (random locations: fp32 SCA).
__device__ __forceinline__ int xcd_chunk(int r, int bps) { return (r & 7) * (bps >> 3) + (r >> 3); }
__device__ __forceinline__ int xcd_block() {
  return (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
}

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

  // block -> (slice, chunk): slices one after the other; within a slice, the blocks of
  // XCD x (block index = x mod 8) take the x-th contiguous eighth of the queries.
  const int slice = blockIdx.x / p.blocks_per_slice;
  const int chunk = xcd_chunk(blockIdx.x - slice * p.blocks_per_slice, p.blocks_per_slice);
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
  lane_group_sum<G, LPU>(acc);

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

// Slice streaming for msda_wave_lds_kernel: the first kStreamBlocks blocks of a (batch,
// head-group) slice each touch one word of every 128-byte value line (one line per
// position) of a 1 / kStreamBlocks share of the slice, in position order, before their own
// units, and throw the words away. With the inputs cold in HBM, the random first touches
// of the slice's gathers then find most lines already in the XCD's L2 or the last-level
// cache: SCA fp32 cold 382.4 -> 375.0 us with full-line loads (32 / 128 / 256 streaming
// blocks: 379.0 / 376.1 / 382.4 us; a share in every block: 425.5 us, too late and too
// much texture-path work; blocks half-way through slice k streaming slice k + 1 instead:
// 375-376 us), and with the record stream below in place one word per line instead of
// full lines 346.8 -> 342.4 us (eight times fewer loads). The price is paid with warm
// inputs: back-to-back launches 318.5 -> 327.0 us. Only slices of at least
// 4 * kStreamBlocks blocks stream. The words are folded into a value stored under a
// condition that never holds, so the loads are kept.
constexpr int kStreamBlocks = 64;

template <typename T, int D>
__device__ __forceinline__ void stream_slice_lines(const WaveParams &p, int b, int hg, int chunk) {
  const uint32_t line = (uint32_t)(p.heads_per_slice * D * sizeof(T));
  if (chunk >= kStreamBlocks || line != 128u || p.blocks_per_slice < 4 * kStreamBlocks) return;
  const __amdgpu_buffer_rsrc_t rs =
      make_rsrc(static_cast<const T *>(p.value) + (int64_t)b * p.S * p.NH * D, p.batch_bytes);
  const int per = (p.S + kStreamBlocks - 1) / kStreamBlocks;
  const int p0 = min(p.S, chunk * per), p1 = min(p.S, p0 + per);
  const uint32_t pos_bytes = (uint32_t)(p.NH * D * sizeof(T)), col = (uint32_t)hg * line;
  uint32_t sink = 0;
  for (int r0 = p0; r0 < p1; r0 += 8 * kBlock) {  // 8 loads in flight per thread
    int v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int pos = r0 + k * kBlock + (int)threadIdx.x;
      v[k] = __builtin_amdgcn_raw_buffer_load_b32(
          rs, pos < p1 ? (uint32_t)pos * pos_bytes + col : p.batch_bytes, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) sink ^= (uint32_t)v[k];
  }
  if (p.NQ < 0 && sink == 0x9e3779b9u) *static_cast<unsigned char *>(p.out) = 0;
}

// The same streaming blocks touch one word of every 128-byte line of their share of the
// slice's sampling-location and attention-weight records (NS samples per (query, head)
// unit), which the slice's blocks read later with non-temporal loads: SCA fp32 cold 369.8
// -> 345.2 us and warm 327.5 -> 298.2 us (with 32 or 128 streaming blocks the same; the
// kernel's own record loads made ordinary instead: 361.1 / 322.2 us).
template <typename T, int NS>
__device__ __forceinline__ void stream_slice_records(const WaveParams &p, int b, int hg,
                                                     int chunk) {
  if (chunk >= kStreamBlocks || p.blocks_per_slice < 4 * kStreamBlocks) return;
  constexpr uint32_t kLoc = NS * 2 * sizeof(T), kAtt = NS * sizeof(T);  // bytes per unit
  constexpr int LL = kLoc >= 128 ? kLoc / 128 : 1, AL = kAtt >= 128 ? kAtt / 128 : 1;
  const int hps = p.heads_per_slice, h0 = hg * hps;
  const int per = (p.NQ + kStreamBlocks - 1) / kStreamBlocks;
  const int q0 = min(p.NQ, chunk * per), q1 = min(p.NQ, q0 + per);
  const int64_t units = (int64_t)p.NQ * p.NH;  // per batch
  // 32-bit ranges: a batch's records past 4 GB read as zeros here (prefetch only)
  const __amdgpu_buffer_rsrc_t lr =
      make_rsrc(static_cast<const T *>(p.loc) + (int64_t)b * units * NS * 2,
                (uint32_t)min<int64_t>(units * kLoc, 0xffffffffll));
  const __amdgpu_buffer_rsrc_t ar =
      make_rsrc(static_cast<const T *>(p.attn) + (int64_t)b * units * NS,
                (uint32_t)min<int64_t>(units * kAtt, 0xffffffffll));
  uint32_t sink = 0;
  const int nl = (q1 - q0) * hps * LL, na = (q1 - q0) * hps * AL;
  for (int i = threadIdx.x; i < nl; i += kBlock) {
    const int line = i % LL, r = i / LL, q = q0 + r / hps, h = h0 + r % hps;
    sink ^= (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
        lr, (uint32_t)(((int64_t)q * p.NH + h) * kLoc) + (uint32_t)line * 128u, 0, 0);
  }
  for (int i = threadIdx.x; i < na; i += kBlock) {
    const int line = i % AL, r = i / AL, q = q0 + r / hps, h = h0 + r % hps;
    sink ^= (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
        ar, (uint32_t)(((int64_t)q * p.NH + h) * kAtt) + (uint32_t)line * 128u, 0, 0);
  }
  if (p.NQ < 0 && sink == 0x9e3779b9u) *static_cast<unsigned char *>(p.out) = 0;
}

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
  const int lblk = xcd_block();  // the slice-major order, XCD x taking its x-th eighth
  const int slice = lblk / p.blocks_per_slice;
  const int chunk = lblk - slice * p.blocks_per_slice;
  const int b = slice / p.slices_per_batch;
  const int hg = slice - b * p.slices_per_batch;
  const int pos_stride = p.NH * D;
  const uint32_t kOOB = p.batch_bytes;
  stream_slice_lines<T, D>(p, b, hg, chunk);
  stream_slice_records<T, NS>(p, b, hg, chunk);

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
  lane_group_sum<G, LPU>(acc);
  if (q < p.NQ && gi == 0) {
    V o;
#pragma unroll
    for (int k = 0; k < VEC; ++k) o.v[k] = from_acc<T>(acc[k]);
    const int64_t unit = ((int64_t)b * p.NQ + q) * p.NH + h;
    // non-temporal: also with the output projection reading the output next, SCA fp32
    // forward + projection measured 461 us against 465 us with ordinary stores
    store_vec_nt<T, VEC>(static_cast<T *>(p.out) + unit * D + c0, o);
  }
}

// ---------------------------------------------------------------------------------------
// LDS-cached kernel. One block of kCachedBlock threads per CU, persistent. Work item = one
// (batch, head) slice (or a query range of it); item i runs on XCD i % 8 and the XCD's
// blocks split its queries, so each XCD's L2 holds one slice at a time. At the start of an
// item the block copies the slice's coarsest levels (whole image rows, coarsest level
// first, as many as fit) into LDS; corners in cached rows are then read from LDS, the rest
// from the value buffer. LDS gathers do not use the vector-memory path (whose throughput
// is set by the number of 128 B lines it serves, not by the bytes used), and the coarse
// levels are exactly the ones each line of which is read by hundreds of samples.
// Within a wave round, iteration `it` covers one level for UPI units, so fully cached
// levels never diverge; invalid corners of a cached level read a zero row of the cache.
constexpr int kLdsBytes = 160 * 1024;               // gfx950 LDS per CU
constexpr uint32_t kLdsFlag = 0x80000000u;          // corner offset names an LDS address

struct CachedParams {
  const void *value;
  const int64_t *shapes;
  const int64_t *lsi;
  const void *loc;
  const void *attn;
  void *out;
  int S, NH, NQ;
  int nitems;            // slices * parts
  int parts;             // query ranges per slice
  int blocks_per_xcd;    // gridDim.x / 8
  int xcd_group;         // XCDs sharing one item (1, 2, 4 or 8)
  int head_pairs;        // 1: an item is a (batch, head pair) slice, the two heads of which
                         // share the 128-byte lines of value (D * sizeof(T) == 64); half of
                         // the item's blocks take each head, so one L2 fill serves both
  uint32_t batch_bytes;  // bytes of value per batch (buffer range; < 2^31)
};

// Level table and cache layout: row 0 of the cache is zeros, then levels from the
// coarsest. Level MIXL keeps as many whole rows as still fit; every other level is cached
// whole or not at all, so its reads take one path for the whole wave. R[l] = cached rows.
template <int NL, int MIXL>
__device__ __forceinline__ void cache_layout(const CachedParams &p, uint32_t row_bytes,
                                             int cache_bytes, int (&H)[NL], int (&W)[NL],
                                             int (&S)[NL], int (&R)[NL], uint32_t (&Off)[NL]) {
  uint32_t used = row_bytes;
#pragma unroll
  for (int l = NL - 1; l >= 0; --l) {
    H[l] = (int)p.shapes[2 * l];
    W[l] = (int)p.shapes[2 * l + 1];
    S[l] = (int)p.lsi[l];
    const int64_t rowb = (int64_t)W[l] * row_bytes;
    int64_t r = (H[l] > 0 && rowb > 0) ? ((int64_t)cache_bytes - used) / rowb : 0;
    if (r > H[l]) r = H[l];
    if (r < 0) r = 0;
    if (l != MIXL && r < H[l]) r = 0;
    R[l] = (int)r;
    Off[l] = used;
    used += (uint32_t)(r * rowb);
  }
}

// The cached kernel's work, compiled per cache layout. FIX = 2: the two coarsest levels
// are cached whole and the others not at all (SCA and DETR in 16-bit types), so each
// level's path is known at compile time and phase 2 is straight-line code whose waits
// name exactly the loads they need (with per-level run-time paths the merge points wait
// for every load of the round before the first blend). FIX = -1: any layout, each level's
// path chosen at run time.
template <typename T, int D, int NL, int NP, int WPB, int UPW, int MIXL, int FIX>
__device__ __forceinline__ void cached_body(const CachedParams &p, unsigned char *cache,
                                            SampleGeo (*geo)[UPW * NL * NP]) {
  using V = Vec<T, 16 / sizeof(T)>;
  constexpr int VEC = 16 / sizeof(T);
  constexpr int G = D / VEC;           // lanes per sample
  constexpr int NS = NL * NP;          // samples per unit
  constexpr int kBlockThreads = WPB * kWave;
  constexpr int kCacheBytes = kLdsBytes - WPB * UPW * NS * (int)sizeof(SampleGeo);
  constexpr int LPL = NP * G;          // lanes per (unit, level)
  constexpr int UPI = kWave / LPL;     // units per iteration
  constexpr int NACC = UPW / UPI;      // accumulator sets per lane
  constexpr int NIT = NL * NACC;       // iterations per round
  constexpr uint32_t ROW = D * sizeof(T);
  static_assert(G >= 1 && UPW * NS <= kWave && LPL <= kWave && kWave % LPL == 0 &&
                    UPW % UPI == 0, "unsupported MSDA geometry");

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  // Block -> (group of xcd_group XCDs, rank in the group). Items of group gi are
  // gi, gi + ngroups, ...; the group's blocks split each item's queries.
  const int xcd = blockIdx.x & 7;
  const int ngroups = 8 / p.xcd_group;
  const int gi = xcd / p.xcd_group;
  const int kb = (xcd - gi * p.xcd_group) * p.blocks_per_xcd + (blockIdx.x >> 3);
  const int nkb = p.xcd_group * p.blocks_per_xcd;
  const int pos_stride = p.NH * D;
  const uint32_t kOOB = p.batch_bytes;

  int lvH[NL], lvW[NL], lvS[NL], lvR[NL];
  uint32_t lvOff[NL];
  cache_layout<NL, MIXL>(p, ROW, kCacheBytes, lvH, lvW, lvS, lvR, lvOff);
  if (threadIdx.x < (int)(ROW / 16)) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<i4 *>(cache + threadIdx.x * 16) = i4{0, 0, 0, 0};
  }

  const int ul = lane & (LPL - 1);
  const int ui = lane / LPL;
  const int pt = ul / G;
  const uint32_t cb = (uint32_t)((ul - pt * G) * VEC * sizeof(T));

  for (int item = gi; item < p.nitems; item += ngroups) {
    int slice = item / p.parts;
    const int part = item - slice * p.parts;
    int kbi = kb, nkbi = nkb;  // this block's rank among the item's blocks for its head
    if (p.head_pairs) {
      const int nlo = nkb / 2, hi = kb >= nlo ? 1 : 0;
      slice = 2 * slice + hi;
      kbi = kb - hi * nlo;
      nkbi = hi ? nkb - nlo : nlo;
    }
    const int b = slice / p.NH;
    const int h = slice - b * p.NH;
    const int qa = (int)((int64_t)p.NQ * part / p.parts);
    const int nqp = (int)((int64_t)p.NQ * (part + 1) / p.parts) - qa;
    const int q0 = qa + (int)((int64_t)nqp * kbi / nkbi);
    const int q1 = qa + (int)((int64_t)nqp * (kbi + 1) / nkbi);
    if (q0 >= q1) continue;  // uniform over the block

    const T *vbase = static_cast<const T *>(p.value) + (int64_t)b * p.S * pos_stride;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(vbase, p.batch_bytes);

    // Fill the cache (the previous item's readers are done after this barrier).
    __syncthreads();
#pragma unroll
    for (int l = NL - 1; l >= 0; --l) {
      const int n16 = lvR[l] * lvW[l] * G;  // 16-byte pieces of this level's cached rows
      const uint32_t src0 = (uint32_t)((lvS[l] * pos_stride + h * D) * sizeof(T));
      for (int i0 = threadIdx.x; i0 < n16; i0 += 4 * kBlockThreads) {
        typedef int i4 __attribute__((ext_vector_type(4)));
        i4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int i = i0 + k * kBlockThreads;
          const int pos = i / G, piece = i - (i / G) * G;
          v[k] = __builtin_amdgcn_raw_buffer_load_b128(
              rsrc, i < n16 ? src0 + (uint32_t)(pos * pos_stride) * sizeof(T) + piece * 16 : kOOB,
              0, 0);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int i = i0 + k * kBlockThreads;
          if (i < n16) *reinterpret_cast<i4 *>(cache + lvOff[l] + (uint32_t)i * 16) = v[k];
        }
      }
    }
    __syncthreads();

    const int nunits = q1 - q0;
    const int64_t unit_base = ((int64_t)b * p.NQ + q0) * p.NH + h;  // unit of query q0
    // Phase-1 inputs of this lane's sample (lanes past UPW * NS repeat lower lanes).
    const int s1 = lane % NS;
    const int u1 = (lane % (UPW * NS)) / NS;
    const int l1 = s1 / NP;
    auto load_in = [&](int u0, float &x, float &y, float &a) {
      const int u = u0 + u1;
      const int uc = u < nunits ? u : nunits - 1;
      const int64_t unit = unit_base + (int64_t)uc * p.NH;
      const T *lp = static_cast<const T *>(p.loc) + (unit * NS + s1) * 2;
      const T *ap = static_cast<const T *>(p.attn) + unit * NS + s1;
      if constexpr (sizeof(T) == 2 && NP == 4) {
        // 16-bit types with 4 points (Deformable DETR): ordinary loads measured faster
        // (100 -> 94 us fp16); streaming loads elsewhere (ordinary: fp32 154 -> 158 us,
        // SCA fp16 255 -> 273 us)
        x = static_cast<float>(lp[0]);
        y = static_cast<float>(lp[1]);
        a = static_cast<float>(*ap);
      } else {
        load_loc<T>(lp, x, y);
        a = static_cast<float>(load_nt(ap));
      }
    };
    // Loads of the next round are issued before this round's gathers (indices clamped,
    // so the loads are unconditional and their registers carry over without a copy).
    float nx, ny, na;
    const bool geo_lane = lane < UPW * NS;
    load_in(wave * UPW, nx, ny, na);

    for (int u0 = wave * UPW; u0 < nunits; u0 += WPB * UPW) {
      const float x = nx, y = ny, a = na;
      load_in(u0 + WPB * UPW, nx, ny, na);
      // Phase 1: lane i computes sample i % NS of unit u0 + i / NS.
      if (geo_lane) {
        int Hl = lvH[0], Wl = lvW[0], Sl = lvS[0], Rl = lvR[0];
        uint32_t Ol = lvOff[0];
#pragma unroll
        for (int i = 1; i < NL; ++i)
          if (l1 == i) { Hl = lvH[i]; Wl = lvW[i]; Sl = lvS[i]; Rl = lvR[i]; Ol = lvOff[i]; }
        const float him = y * (float)Hl - 0.5f, wim = x * (float)Wl - 0.5f;
        // Invalid corners: the zero row when the level is cached, else out of range.
        const uint32_t zero = Rl > 0 ? kLdsFlag : kOOB;
        SampleGeo sg;
        sg.w[0] = sg.w[1] = sg.w[2] = sg.w[3] = 0.f;
        sg.o[0] = sg.o[1] = sg.o[2] = sg.o[3] = zero;
        if (u0 + u1 < nunits && him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl) {
          const float fh = floorf(him), fw = floorf(wim);
          const int hl = (int)fh, wl = (int)fw;
          const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
          const bool y0 = hl >= 0, y1 = hl + 1 <= Hl - 1, x0 = wl >= 0, x1 = wl + 1 <= Wl - 1;
          auto corner = [&](int yy, int xx) -> uint32_t {
            if (yy < Rl) return kLdsFlag | (Ol + (uint32_t)(yy * Wl + xx) * ROW);
            return (uint32_t)(((Sl + yy * Wl + xx) * pos_stride + h * D) * sizeof(T));
          };
          if (y0 && x0) { sg.w[0] = hh * hw * a; sg.o[0] = corner(hl, wl); }
          if (y0 && x1) { sg.w[1] = hh * lw * a; sg.o[1] = corner(hl, wl + 1); }
          if (y1 && x0) { sg.w[2] = lh * hw * a; sg.o[2] = corner(hl + 1, wl); }
          if (y1 && x1) { sg.w[3] = lh * lw * a; sg.o[3] = corner(hl + 1, wl + 1); }
        }
        geo[wave][lane] = sg;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // Phase 2: iteration it gathers level it % NL of units (it / NL) * UPI + ui. All
      // geometry reads first, then every corner load, then the arithmetic.
      SampleGeo sg[NIT];
#pragma unroll
      for (int it = 0; it < NIT; ++it)
        sg[it] = geo[wave][((it / NL) * UPI + ui) * NS + (it % NL) * NP + pt];
      V v[NIT][4];
      V vx[NACC][4];  // level MIXL: the value-buffer half of a cached-in-part level
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int l = it % NL;
        if (FIX < 0 && l == MIXL && lvR[l] > 0 && lvR[l] < lvH[l]) {
          // Each corner is in the cache or in the value buffer; the other read returns 0.
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const uint32_t o = sg[it].o[c];
            const bool in_lds = (o & kLdsFlag) != 0;
            v[it][c] = *reinterpret_cast<const V *>(cache + (in_lds ? (o & ~kLdsFlag) + cb : cb));
            vx[it / NL][c] = buffer_load_vec<T, VEC>(rsrc, in_lds ? kOOB : o + cb);
          }
        } else if (FIX >= 0 ? l >= NL - FIX : lvR[l] > 0) {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v[it][c] = *reinterpret_cast<const V *>(cache + ((sg[it].o[c] & ~kLdsFlag) + cb));
            if (FIX < 0 && l == MIXL) vx[it / NL][c] = V{};
          }
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            v[it][c] = buffer_load_vec<T, VEC>(rsrc, sg[it].o[c] + cb);
            if (FIX < 0 && l == MIXL) vx[it / NL][c] = V{};
          }
        }
      }
      if constexpr (MIXL >= 0 && FIX < 0) {
        // One of each pair is all-zero bits: OR keeps the other exactly.
#pragma unroll
        for (int it = MIXL; it < NIT; it += NL)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            typedef int i4 __attribute__((ext_vector_type(4)));
            v[it][c] = __builtin_bit_cast(V, __builtin_bit_cast(i4, v[it][c]) |
                                                 __builtin_bit_cast(i4, vx[it / NL][c]));
          }
      }
      float acc[NACC][VEC];
#pragma unroll
      for (int a = 0; a < NACC; ++a)
#pragma unroll
        for (int k = 0; k < VEC; ++k) acc[a][k] = 0.f;
#pragma unroll
      for (int it = 0; it < NIT; ++it)
#pragma unroll
        for (int k = 0; k < VEC; ++k) {
          float t = acc[it / NL][k];
          t += sg[it].w[0] * (float)v[it][0].v[k];
          t += sg[it].w[1] * (float)v[it][1].v[k];
          t += sg[it].w[2] * (float)v[it][2].v[k];
          t += sg[it].w[3] * (float)v[it][3].v[k];
          acc[it / NL][k] = t;
        }
      // Sum over the points of each (unit, level) lane block.
      lane_group_sum<G, LPL>(*reinterpret_cast<float (*)[NACC * VEC]>(&acc[0][0]));
      if (pt == 0) {
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
          const int u = u0 + a * UPI + ui;
          if (u < nunits) {
            V o;
#pragma unroll
            for (int k = 0; k < VEC; ++k) o.v[k] = from_acc<T>(acc[a][k]);
            // ordinary stores: the output projection reads the output next and finds it
            // in the cache (DETR fp32 forward + projection 214.6 -> 205.5 us against
            // non-temporal stores; the forward alone is 0-4 us slower)
            store_vec<T, VEC>(static_cast<T *>(p.out) + (unit_base + (int64_t)u * p.NH) * D +
                                  cb / sizeof(T),
                              o);
          }
        }
      }
      // The next round rewrites this wave's geometry slots.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// WPB waves per block, UPW (b, q, head) units per wave round, MIXL the one level that may
// be cached in part (-1: none). The layout check is uniform over the grid. The fixed-layout
// body is compiled for 16-bit types (SCA fp16 239.9 -> 237.7 us, bf16 252.0 -> 243.4 us,
// DETR bf16 93.1 -> 91.2 us), the only ones the dispatch sends here; the run-time body
// serves any layout.
template <typename T, int D, int NL, int NP, int WPB, int UPW, int MIXL>
__global__ void __launch_bounds__(WPB * kWave) msda_cached_kernel(const CachedParams p) {
  constexpr int kCacheBytes = kLdsBytes - WPB * UPW * NL * NP * (int)sizeof(SampleGeo);
  __shared__ __attribute__((aligned(16))) unsigned char cache[kCacheBytes];
  __shared__ SampleGeo geo[WPB][UPW * NL * NP];
  if constexpr (sizeof(T) == 2 && NL >= 2) {
    int H[NL], W[NL], S[NL], R[NL];
    uint32_t Off[NL];
    cache_layout<NL, MIXL>(p, D * sizeof(T), kCacheBytes, H, W, S, R, Off);
    bool fixed = true;
#pragma unroll
    for (int l = 0; l < NL; ++l)
      fixed = fixed && (l >= NL - 2 ? H[l] > 0 && W[l] > 0 && R[l] == H[l] : R[l] == 0);
    if (fixed) {
      cached_body<T, D, NL, NP, WPB, UPW, MIXL, 2>(p, cache, geo);
      return;
    }
  }
  cached_body<T, D, NL, NP, WPB, UPW, MIXL, -1>(p, cache, geo);
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
  p.blocks_per_slice =
      (int)((units_per_slice + units_per_block - 1) / units_per_block + 7) & ~7;
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

int gcd_int(int x, int y) {
  while (y) { const int t = x % y; x = y; y = t; }
  return x;
}

// The cached kernel pays one LDS fill per (item, block); it is used when every block
// has a few hundred units per item and there is more than one level to cache.
template <typename T, int D, int NL, int NP>
bool cached_worthwhile(const MsdaArgs &a) {
  const int cus = device_cus();
  if (NL < 2 || cus < 8) return false;
  const int64_t units = (int64_t)a.batch * a.num_heads * a.num_query;
  return units >= (int64_t)cus * 256;
}

// UPW_MIN: wanted units per wave round, raised to a whole iteration's units.
template <typename T, int D, int NL, int NP, int WPB, int UPW_MIN, int MIXL = NL - 2>
hipError_t launch_cached_t(const MsdaArgs &a, hipStream_t stream, int xcd_group = 1) {
  constexpr int UPI = kWave / (NP * (D / (16 / (int)sizeof(T))));
  constexpr int UPW = UPW_MIN > UPI ? UPW_MIN : UPI;
  CachedParams p;
  p.value = a.value;
  p.shapes = a.spatial_shapes;
  p.lsi = a.level_start_index;
  p.loc = a.sampling_loc;
  p.attn = a.attn_weight;
  p.out = a.output;
  p.S = a.spatial_size;
  p.NH = a.num_heads;
  p.NQ = a.num_query;
  const int blocks = (device_cus() / 8) * 8;
  p.blocks_per_xcd = blocks / 8;
  p.xcd_group = xcd_group;
  // 16-bit D = 32: two heads per 128-byte line; items are head pairs when every block of
  // the item's XCD group has a partner for the other head
  p.head_pairs = (D * (int)sizeof(T) == 64 && a.num_heads % 2 == 0 &&
                  p.blocks_per_xcd * xcd_group >= 2) ? 1 : 0;
  const int slices = a.batch * a.num_heads / (p.head_pairs ? 2 : 1);
  p.parts = 8 / gcd_int(slices, 8);  // items = a multiple of the 8 XCDs
  p.nitems = slices * p.parts;
  p.batch_bytes = (uint32_t)((int64_t)a.spatial_size * a.num_heads * D * sizeof(T));
  if (blocks == 0 || p.nitems == 0) return hipSuccess;
  hipLaunchKernelGGL((msda_cached_kernel<T, D, NL, NP, WPB, UPW, MIXL>), dim3(blocks),
                     dim3(WPB * kWave), 0, stream, p);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------------------
// Tiled single-level kernel for self-attention over one grid (BEVFormer temporal
// self-attention): one level, num_query == H * W, query q being cell (q / W, q % W), and
// each query samples near its own cell. Work item = (batch, head, TS x TS tile of query
// cells). The block copies the tile's neighbourhood (the tile grown by MG cells on every
// side) of the head's value rows into LDS once, and every corner inside it is read from
// there; a corner outside it is read from the value buffer in a branch taken only when
// some lane of the wave needs it. When the shapes do not describe the queries
// (H * W != num_query) the kernel takes the queries in index order and reads every corner
// from the value buffer. Persistent blocks; each XCD takes a contiguous range of items, so
// neighbouring tiles (which share neighbourhood rows) meet in its L2.
struct TileParams {
  const void *value;
  const int64_t *shapes;
  const int64_t *lsi;
  const void *loc;
  const void *attn;
  void *out;
  int B, S, NH, NQ;
  int blocks_per_xcd;    // gridDim.x / 8
  uint32_t batch_bytes;  // bytes of value per batch (< 2^31)
};

// BPC workgroups of WPB waves per CU: the second bound is waves per SIMD.
// PF: the next item's locations, weights and neighbourhood are loaded into registers
// while the current item's passes run (the registers must allow it: 16-bit types).
template <typename T, int NP, int TS, int MG, int WPB, int BPC, bool PF>
__global__ void __launch_bounds__(WPB * kWave, (WPB * BPC + 3) / 4) msda_tile_kernel(const TileParams p) {
  constexpr int D = 32;
  constexpr int VEC = 16 / (int)sizeof(T);
  using V = Vec<T, VEC>;
  constexpr int G = D / VEC;             // lanes per corner
  constexpr int NG = kWave / G;          // lane groups per wave
  constexpr int RS = TS + 2 * MG;        // neighbourhood side
  constexpr uint32_t ROW = D * sizeof(T);
  constexpr uint32_t kRegion = RS * RS * ROW;
  constexpr int UPP = kWave / NP;        // units per geometry pass (one sample per lane)
  constexpr int UPG = UPP / NG;          // units per lane group and pass
  constexpr int NPASS = (TS * TS + WPB * UPP - 1) / (WPB * UPP);  // geometry passes per wave
  static_assert(kWave % NP == 0 && UPP % NG == 0 && UPG >= 1, "unsupported tile geometry");
  __shared__ __attribute__((aligned(16))) unsigned char region[kRegion + ROW];  // + zero row
  __shared__ SampleGeo geo[WPB][kWave];   // weights, LDS byte address of every corner
  __shared__ uint4 far_off[WPB][kWave];    // value-buffer offsets of corners outside it

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int H = (int)p.shapes[0], W = (int)p.shapes[1], S0 = (int)p.lsi[0];
  const bool grid = (int64_t)H * W == p.NQ && H > 0 && W > 0;
  const int tiles_x = grid ? (W + TS - 1) / TS : 1;
  const int ntile = grid ? tiles_x * ((H + TS - 1) / TS) : (p.NQ + TS * TS - 1) / (TS * TS);
  const int nitems = p.B * p.NH * ntile;
  const int xcd = blockIdx.x & 7;
  const int per = (nitems + 7) / 8;
  const int i_end = min(nitems, (xcd + 1) * per);
  const int pos_stride = p.NH * D;
  const uint32_t kOOB = p.batch_bytes;
  const float Hf = (float)H, Wf = (float)W;
  if (threadIdx.x < (int)(ROW / 16)) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    *reinterpret_cast<i4 *>(region + kRegion + threadIdx.x * 16) = i4{0, 0, 0, 0};
  }
  const int g = lane / G;
  const uint32_t cb = (uint32_t)(lane % G) * 16u;

  typedef int i4 __attribute__((ext_vector_type(4)));
  constexpr int P16 = ROW / 16;
  constexpr int NPC = RS * RS * P16;              // 16-byte pieces of the neighbourhood
  constexpr int NT = WPB * kWave;
  constexpr int NLD = (NPC + NT - 1) / NT;        // pieces per thread
  // Query of unit ul of tile `tile` = (ty, tx) (valid flag in qv).
  auto query_of = [&](int tile, int ty, int tx, int ul, bool &qv)
      __attribute__((always_inline)) -> int {
    if (grid) {
      const int qy = ty * TS + ul / TS, qx = tx * TS + ul % TS;
      qv = ul < TS * TS && qy < H && qx < W;
      return qy * W + qx;
    }
    const int q = tile * TS * TS + ul;
    qv = ul < TS * TS && q < p.NQ;
    return q;
  };
  // Loads of item `it`: this wave's locations and weights of the tile, and the thread's
  // pieces of the head's value rows of the tile grown by MG cells on every side (out of
  // range, i.e. no request, past the grid, past the last item or without a grid). Every
  // load is unconditional, so the wait counts stay exact.
  float lx[NPASS], ly[NPASS], la[NPASS];
  i4 v[NLD];
  auto fetch_loc = [&](int tile, int ty, int tx, int b, int h) __attribute__((always_inline)) {
    // every pass's address first, then the loads: address arithmetic between the loads
    // let the register allocator put a temporary on a pending load's register, which
    // cost a wait for the first pass's loads before the second's were issued
    const T *lp[NPASS];
    const T *ap[NPASS];
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      bool qv;
      const int q = query_of(tile, ty, tx, (wave + ps * WPB) * UPP + lane / NP, qv);
      const int64_t unit = ((int64_t)b * p.NQ + (qv ? q : 0)) * p.NH + h;
      lp[ps] = static_cast<const T *>(p.loc) + (unit * NP + lane % NP) * 2;
      ap[ps] = static_cast<const T *>(p.attn) + unit * NP + lane % NP;
    }
    // ordinary loads here (the other kernels stream these inputs): measured 98.4 ->
    // 94.0 us for the temporal self-attention map, whose tiles' rows stay in L2
#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      lx[ps] = static_cast<float>(lp[ps][0]);
      ly[ps] = static_cast<float>(lp[ps][1]);
      la[ps] = static_cast<float>(*ap[ps]);
    }
  };
  // neighbourhood with origin (ry0, rx0) of head offset hof in the batch slice rs
  auto fetch_nb = [&](bool live, int ry0, int rx0, __amdgpu_buffer_rsrc_t rs, uint32_t hof)
      __attribute__((always_inline)) {
#pragma unroll
    for (int k = 0; k < NLD; ++k) {
      const int i = (int)threadIdx.x + k * NT;
      const int pos = i / P16, piece = i - pos * P16;
      const int y = ry0 + pos / RS, x = rx0 + pos % RS;
      const bool in = live && i < NPC && (unsigned)y < (unsigned)H && (unsigned)x < (unsigned)W;
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(
          rs, in ? (uint32_t)((S0 + y * W + x) * pos_stride) * sizeof(T) + hof + piece * 16
                 : kOOB,
          0, 0);
    }
  };

  // PF: the loads of item it (past the last item: locations of the last, no neighbourhood)
  auto fetch_item = [&](int it) __attribute__((always_inline)) {
    const bool live = grid && it < i_end;
    const int itc = it < i_end ? it : i_end - 1;  // a valid item for the location reads
    const int tile = itc % ntile, bh = itc / ntile;
    const int h = bh % p.NH, b = bh / p.NH;
    const int ty = tile / tiles_x, tx = tile - ty * tiles_x;
    fetch_loc(tile, ty, tx, b, h);
    fetch_nb(live, ty * TS - MG, tx * TS - MG,
             make_rsrc(static_cast<const T *>(p.value) + (int64_t)b * p.S * pos_stride,
                       p.batch_bytes),
             (uint32_t)(h * D * sizeof(T)));
  };
  int item = xcd * per + (blockIdx.x >> 3);
  if constexpr (PF) {
    if (item >= i_end) return;  // (fetch_item needs an item of this block)
    fetch_item(item);
  }
  for (; item < i_end; item += p.blocks_per_xcd) {
    // without PF (fp32, whose registers are taken): locations first, the neighbourhood
    // after the barrier below, every load of the item in flight before the first store
    const int tile = item % ntile;
    const int bh = item / ntile;
    const int h = bh % p.NH, b = bh / p.NH;
    const int ty = tile / tiles_x, tx = tile - ty * tiles_x;
    if constexpr (!PF) fetch_loc(tile, ty, tx, b, h);
    // Neighbourhood origin; a huge origin when there is no grid keeps every corner out.
    const int ry0 = grid ? ty * TS - MG : -(1 << 28), rx0 = grid ? tx * TS - MG : -(1 << 28);
    const T *vbase = static_cast<const T *>(p.value) + (int64_t)b * p.S * pos_stride;
    const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(vbase, p.batch_bytes);
    const uint32_t hoff = (uint32_t)(h * D * sizeof(T));
    auto query = [&](int ul, bool &qv) __attribute__((always_inline)) -> int {
      return query_of(tile, ty, tx, ul, qv);
    };
    // this item's locations and weights (PF: copied before the next item's loads reuse
    // lx / ly / la; without PF they are read in place, so nothing waits for them before
    // phase 1)
    float cx[NPASS], cy[NPASS], ca[NPASS];
    if constexpr (PF) {
#pragma unroll
      for (int ps = 0; ps < NPASS; ++ps) {
        cx[ps] = lx[ps];
        cy[ps] = ly[ps];
        ca[ps] = la[ps];
      }
    }

    __syncthreads();  // the previous item's readers are done
    if (PF || grid) {
      if constexpr (!PF) fetch_nb(true, ry0, rx0, rsrc, hoff);
#pragma unroll
      for (int k = 0; k < NLD; ++k) {
        const int i = (int)threadIdx.x + k * NT;
        if (i < NPC) *reinterpret_cast<i4 *>(region + (uint32_t)i * 16) = v[k];
      }
    }
    __syncthreads();
    // the next item's loads, in flight during this item's passes
    if constexpr (PF) fetch_item(item + p.blocks_per_xcd);

#pragma unroll
    for (int ps = 0; ps < NPASS; ++ps) {
      const int u0 = (wave + ps * WPB) * UPP;
      if (u0 >= TS * TS) break;  // uniform over the wave
      // Phase 1: lane = (unit u0 + lane / NP, point lane % NP).
      bool far;  // some corner of the pass lies outside the neighbourhood
      {
        bool qv;
        query(u0 + lane / NP, qv);
        const float x = PF ? cx[ps] : lx[ps], y = PF ? cy[ps] : ly[ps], a = PF ? ca[ps] : la[ps];
        const float him = y * Hf - 0.5f, wim = x * Wf - 0.5f;
        // Corners inside the neighbourhood: their LDS address; outside it (or invalid):
        // the zero row, and for a valid one its value-buffer offset in far_off. Written
        // with selects (no per-corner branches), so every array index stays constant.
        SampleGeo sg;
        uint32_t fo[4];
        const bool in = qv && him > -1.f && wim > -1.f && him < Hf && wim < Wf;
        const float fh = floorf(him), fw = floorf(wim);
        const int hl = (int)fh, wl = (int)fw;
        const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int yy = hl + (c >> 1), xx = wl + (c & 1);
          const bool ok = in && (unsigned)yy < (unsigned)H && (unsigned)xx < (unsigned)W;
          const int ry = yy - ry0, rx = xx - rx0;
          const bool near = (unsigned)ry < (unsigned)RS && (unsigned)rx < (unsigned)RS;
          const float wy = (c >> 1) ? lh : hh, wx = (c & 1) ? lw : hw;
          sg.w[c] = ok ? wy * wx * a : 0.f;
          sg.o[c] = ok && near ? (uint32_t)(ry * RS + rx) * ROW : kRegion;
          fo[c] = ok && !near ? (uint32_t)((S0 + yy * W + xx) * pos_stride) * sizeof(T) + hoff
                              : kOOB;
        }
        far_off[wave][lane] = uint4{fo[0], fo[1], fo[2], fo[3]};
        far = __builtin_amdgcn_ballot_w64(fo[0] != kOOB || fo[1] != kOOB || fo[2] != kOOB ||
                                          fo[3] != kOOB) != 0;
        geo[wave][lane] = sg;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // Phase 2: lane group g sums the NP samples of units g, g + NG, ... in registers.
#pragma unroll
      for (int k = 0; k < UPG; ++k) {
        const int uu = g + NG * k;
        SampleGeo sg[NP];
#pragma unroll
        for (int s = 0; s < NP; ++s) sg[s] = geo[wave][uu * NP + s];
        V v[NP][4];
#pragma unroll
        for (int s = 0; s < NP; ++s)
#pragma unroll
          for (int c = 0; c < 4; ++c)
            v[s][c] = *reinterpret_cast<const V *>(region + (sg[s].o[c] + cb));
        if (far) {
          // Corners outside the neighbourhood: the LDS read above returned zero bits.
#pragma unroll
          for (int s = 0; s < NP; ++s) {
            const uint4 fo = far_off[wave][uu * NP + s];
            const uint32_t fa[4] = {fo.x, fo.y, fo.z, fo.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const V f = buffer_load_vec<T, VEC>(rsrc, fa[c] + cb);
              typedef int i4 __attribute__((ext_vector_type(4)));
              v[s][c] = __builtin_bit_cast(V, __builtin_bit_cast(i4, v[s][c]) |
                                                  __builtin_bit_cast(i4, f));
            }
          }
        }
        float acc[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
#pragma unroll
        for (int s = 0; s < NP; ++s)
#pragma unroll
          for (int e = 0; e < VEC; ++e) {
            float t = acc[e];
            t += sg[s].w[0] * (float)v[s][0].v[e];
            t += sg[s].w[1] * (float)v[s][1].v[e];
            t += sg[s].w[2] * (float)v[s][2].v[e];
            t += sg[s].w[3] * (float)v[s][3].v[e];
            acc[e] = t;
          }
        bool qv;
        const int q = query(u0 + uu, qv);
        if (qv) {
          V o;
#pragma unroll
          for (int e = 0; e < VEC; ++e) o.v[e] = from_acc<T>(acc[e]);
          // ordinary stores, for the reader of the output (TSA fp16 forward + projection
          // 101.3 -> 95.9 us against non-temporal stores; the forward alone +2.3 us)
          store_vec<T, VEC>(static_cast<T *>(p.out) +
                                (((int64_t)b * p.NQ + q) * p.NH + h) * D + (lane % G) * VEC,
                            o);
        }
      }
      // The next pass rewrites this wave's geometry.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }
}

// BPC: workgroups per CU (the LDS use must allow it).
template <typename T, int NP, int TS, int MG, int WPB, int BPC, bool PF>
hipError_t launch_tile_t(const MsdaArgs &a, hipStream_t stream) {
  TileParams p;
  p.value = a.value;
  p.shapes = a.spatial_shapes;
  p.lsi = a.level_start_index;
  p.loc = a.sampling_loc;
  p.attn = a.attn_weight;
  p.out = a.output;
  p.B = a.batch;
  p.S = a.spatial_size;
  p.NH = a.num_heads;
  p.NQ = a.num_query;
  const int blocks = (device_cus() / 8) * 8 * BPC;
  p.blocks_per_xcd = blocks / 8;
  p.batch_bytes = (uint32_t)((int64_t)a.spatial_size * a.num_heads * 32 * sizeof(T));
  if (blocks == 0 || a.batch == 0 || a.num_query == 0) return hipSuccess;
  hipLaunchKernelGGL((msda_tile_kernel<T, NP, TS, MG, WPB, BPC, PF>), dim3(blocks),
                     dim3(WPB * kWave), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_wave(const MsdaArgs &a, hipStream_t stream) {
  const int L = a.num_levels, P = a.num_point;
  switch (a.channels) {
    case 32:
      if (L == 4 && P == 8) {  // BEVFormer SCA
        // fp32: the per-sample gather kernel at high occupancy measured faster than the
        // cached kernel (whose partly cached level still costs a load per corner).
        if constexpr (sizeof(T) == 2)
          if (cached_worthwhile<T, 32, 4, 8>(a)) return launch_cached_t<T, 32, 4, 8, 12, 2>(a, stream);
        return launch_wave_t<T, 32, 4, 8>(a, stream);
      }
      if (L == 1 && P == 4) {  // BEVFormer TSA
        // the tiled kernel (neighbourhood in LDS) measured faster than the per-sample
        // gather kernel: fp32 by 25%, fp16 74.0 -> 69.1 us, bf16 75.4 -> 73.6 us
        if (a.num_query == a.spatial_size && device_cus() >= 8) {
          if constexpr (sizeof(T) == 2)
            return launch_tile_t<T, 4, 16, 6, 8, 1, true>(a, stream);
          else
            return launch_tile_t<T, 4, 16, 6, 8, 1, false>(a, stream);
        }
        return launch_wave_t<T, 32, 1, 4>(a, stream);
      }
      if (L == 4 && P == 4) {  // Deformable DETR
        // 16-bit types: the LDS-cached kernel. fp32: the per-sample kernel, whose slice
        // streaming (value lines and records) measured DETR fp32 cold 154.9 -> 152.8 us and
        // warm 138.6 -> 132.2 us against the cached kernel (fp16: 119.6 against 87.7 us).
        if constexpr (sizeof(T) == 2)
          if (cached_worthwhile<T, 32, 4, 4>(a)) return launch_cached_t<T, 32, 4, 4, 12, 2>(a, stream);
        return launch_wave_t<T, 32, 4, 4>(a, stream);
      }
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

// CU count of the current device, read once per device. Several host threads may launch
// at once: each slot is an atomic, and two threads that both find it empty store the same
// value.
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace bevk
