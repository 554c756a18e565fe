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
//
// D = 32 with fp32 accumulation (every BEVFormer and DETR shape) and a workspace of
// msda_backward_workspace_bytes takes the sorted path (the msda_bkt_* kernels and
// msda_coord_kernel below): the corner adds are bucketed by position and each bucket is
// summed by the workgroup that owns its grad_value rows, so no corner takes an atomic.
// With a smaller workspace, D = 32 runs the per-unit mapping in msda_col2im_d32_kernel
// (32-bit offsets, branch-free corner loads, shorter reduction), and the levels of at most
// kCoarseBins positions leave its atomics for msda_coarse_gv_kernel, which sums each
// position's corner adds of 256 queries before one atomic per channel.
//
// One-level maps whose queries are the grid cells (temporal self-attention) take two other
// kernels below when the sorted path's workspace is not given: msda_gv_owner_kernel adds
// each grad_value row once per position owner, without atomics, and
// msda_grid_coord_kernel computes grad_sampling_loc / grad_attn_weight and adds the
// samples far from their query with atomics.
#include "bevk_common.h"
#include "bevk_launch.h"

#include <hip/amd_detail/amd_hip_unsafe_atomics.h>

#include <algorithm>
#include <type_traits>

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
  int coarse;  // msda_coarse_gv_kernel adds the coarse levels' grad_value (see below)
};

// Coarse levels: the longest run of final levels (l = LC .. NL - 1, stored one after the
// other) whose positions number at most kCoarseBins. Both kernels of the coarse split
// derive LC from the shapes with this function, so every sample is added by exactly one.
constexpr int kCoarseBins = 2048;
__device__ __forceinline__ int coarse_first_level(const int64_t *shapes, const int64_t *lsi,
                                                  int NL, int S) {
  int lc = NL;
  int64_t end = 0;
  for (int l = NL - 1; l >= 0; --l) {
    const int64_t n = shapes[2 * l] * shapes[2 * l + 1];
    if (l == NL - 1) {
      if (lsi[l] < 0 || lsi[l] + n > S) break;
      end = lsi[l] + n;
    } else if (lsi[l] < 0 || lsi[l] + n != lsi[l + 1]) {
      break;
    }
    if (end - lsi[l] > kCoarseBins) break;
    lc = l;
  }
  return lc;
}

// Sampling coordinates of a sample, as fused multiply-adds so that every kernel that
// classifies samples gets the same bits.
template <typename A>
__device__ __forceinline__ void sample_coords(A lx, A ly, int Hl, int Wl, A &him, A &wim) {
  him = fma(ly, (A)Hl, (A)-0.5);
  wim = fma(lx, (A)Wl, (A)-0.5);
}

// One-level grids whose queries are the grid cells (q = y * W + x): a sample is "near"
// when all four of its corners lie within kOwnMargin cells of its query's cell (qy, qx).
// The owner pass adds near samples to grad_value without atomics; the others are added
// by msda_grid_coord_kernel.
constexpr int kOwnMargin = 6;
__device__ __forceinline__ bool near_cell(int hl, int wl, int qy, int qx) {
  return hl >= qy - kOwnMargin && hl + 1 <= qy + kOwnMargin && wl >= qx - kOwnMargin &&
         wl + 1 <= qx + kOwnMargin;
}

// The one level is a grid of exactly num_query cells starting at position 0, so query q
// is cell (q / W, q % W). The owner and the coordinate kernels both read this from the
// device metadata (the host checks only num_level == 1 and num_query == spatial_size);
// when it does not hold, every sample takes the atomic path.
__device__ __forceinline__ bool grid_queries(const int64_t *shapes, const int64_t *lsi, int nq) {
  return shapes[0] * shapes[1] == (int64_t)nq && lsi[0] == 0;
}

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
  const int LC = p.coarse ? coarse_first_level(p.shapes, p.lsi, p.NL, p.S) : p.NL;
  for (int l = 0; l < p.NL; ++l) {
    const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
    const int64_t base = p.lsi[l];
    const bool add = l < LC;  // coarse levels: msda_coarse_gv_kernel
    for (int pt = 0; pt < p.NP; ++pt) {
      const int s = l * p.NP + pt;
      const A lx = (A)lp[2 * s], ly = (A)lp[2 * s + 1], a = (A)ap[s];
      A him, wim;
      sample_coords<A>(lx, ly, Hl, Wl, him, wim);
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
          if (live && add) {
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

// ---------------------------------------------------------------------------
// grad_value without atomics for one-level grids whose queries are the grid cells
// (BEVFormer temporal self-attention: q = y * W + x, D = 32, P <= 4). A persistent
// workgroup owns kOwnT x kOwnT positions of one (batch, head) slice at a time and stores
// their grad_value rows once, without atomics (fp32 grad_value: added to what it holds;
// the fp32 workspace of the 16-bit types: written):
//   1. the candidate queries (cells within kOwnMargin of the tile) have their locations
//      and attention weights loaded, all in flight together; every candidate sample that
//      is near its query (all corners within kOwnMargin cells) and in the window
//      (-1, H) x (-1, W) counts one pair for each of its corners inside the tile and the
//      image (integer LDS atomic, whose result is the pair's rank in its position);
//   2. a scan of the counts gives each position's range, and each corner kept from step 1
//      (position, rank) stores its pair (query, bilinear weight x attention) there;
//   3. each half-wave (32 lanes, one channel each) owns half a tile row: for each
//      position it sums weight x grad_output row of the pair's query over the position's
//      pairs (rows read from L2, 8 in flight) and stores it.
// A tile with more than kOwnCap pairs zeroes its rows and adds its pairs with atomics.
// Every near sample's corner is found by exactly one owner (its query lies within
// kOwnMargin of the corner, so among that tile's candidates); msda_grid_coord_kernel then
// adds the remaining samples with atomics.
// ---------------------------------------------------------------------------
constexpr int kOwnT = 8;
constexpr int kOwnThreads = 512;
constexpr int kOwnSide = kOwnT + 2 * kOwnMargin;              // candidate query side
constexpr int kOwnCand = kOwnSide * kOwnSide;
constexpr int kOwnMaxP = 4;                                   // points per query
// Pairs kept in LDS per tile: a tile of TSA-like data holds about 16 per position (4
// points x 4 corners of ~one query per cell); a tile beyond this adds its pairs with
// atomics instead (see the overflow branch).
constexpr int kOwnCap = 2560;
constexpr int kOwnBins = kOwnT * kOwnT;
static_assert(kOwnBins == kWave, "one wave scans the position counts");
static_assert(kOwnCand * kOwnMaxP * 4 < 65536, "a corner's rank in its position fits 16 bits");

struct OwnParams {
  const void *loc, *attn, *grad_out;
  float *gv;       // grad_value (fp32) or the fp32 workspace of the 16-bit types
  int accumulate;  // add to gv (fp32 grad_value, whose contract is accumulation) or write it
  const int64_t *shapes, *lsi;
  int64_t go_sb, go_sq, go_sh, go_sc;
  int B, NH, NQ, NP, S;
  int blocks_per_xcd;
};

template <typename T, int NP>
__global__ void __launch_bounds__(kOwnThreads) msda_gv_owner_kernel(const OwnParams p) {
  constexpr int D = 32;
  constexpr int kIter = (kOwnCand * NP + kOwnThreads - 1) / kOwnThreads;
  __shared__ int bin_at[kOwnBins + 1];   // counts, then each position's first pair
  __shared__ int lq[kOwnCap];      // pair: query
  __shared__ float lw[kOwnCap];    // pair: bilinear weight x attention
  const int H = (int)p.shapes[0], W = (int)p.shapes[1];
  const int tid = threadIdx.x;
  if (!grid_queries(p.shapes, p.lsi, p.NQ)) {
    // The shapes do not describe the queries as grid cells: no sample is near, so
    // msda_grid_coord_kernel adds every sample with atomics; in write mode the workspace
    // is cleared here first (this kernel runs before it on the same stream).
    if (!p.accumulate) {
      const int64_t n = (int64_t)p.B * p.S * p.NH * 32;
      for (int64_t i = (int64_t)blockIdx.x * kOwnThreads + tid; i < n;
           i += (int64_t)gridDim.x * kOwnThreads)
        p.gv[i] = 0.f;
    }
    return;
  }
  const int tiles_x = (W + kOwnT - 1) / kOwnT;
  const int ntile = tiles_x * ((H + kOwnT - 1) / kOwnT);
  const int nitems = p.B * p.NH * ntile;
  const int xcd = blockIdx.x & 7;
  const int per = (nitems + 7) / 8;
  const int i_end = min(nitems, (xcd + 1) * per);
  const int wave = tid / kWave, half = (tid & (kWave - 1)) >> 5, ch = tid & 31;
  const T *loc = static_cast<const T *>(p.loc);
  const T *attn = static_cast<const T *>(p.attn);
  const T *gout = static_cast<const T *>(p.grad_out);
  for (int item = xcd * per + (blockIdx.x >> 3); item < i_end; item += p.blocks_per_xcd) {
    const int tile = item % ntile;
    const int bh = item / ntile;
    const int h = bh % p.NH, b = bh / p.NH;
    const int ty = tile / tiles_x, tx = tile - ty * tiles_x;
    const int y0 = ty * kOwnT, x0 = tx * kOwnT;
    const int cy0 = max(0, y0 - kOwnMargin), cy1 = min(H, y0 + kOwnT + kOwnMargin);
    const int cx0 = max(0, x0 - kOwnMargin), cx1 = min(W, x0 + kOwnT + kOwnMargin);
    const int cw = cx1 - cx0;
    const int ncand = (cy1 - cy0) * cw;
    const int nsamp = ncand * NP;
    const float inv_cw = 1.f / (float)cw;
    // Candidate c = row * cw + col of the (cy1 - cy0) x cw block (c < 2^10: the rounded
    // float quotient is exact).
    auto cand_row = [&](int c) { return (int)(((float)c + 0.5f) * inv_cw); };
    // Loads of the item, all in flight together: the thread's candidate samples
    // i = tid + k * kOwnThreads (locations, attention).
    float slx[kIter], sly[kIter], sa[kIter];
    int scy[kIter], scx[kIter];
#pragma unroll
    for (int k = 0; k < kIter; ++k) {
      const int i = min(tid + k * kOwnThreads, nsamp - 1);
      const int c = i / NP, pt = i - (i / NP) * NP;
      const int cr = cand_row(c);
      scy[k] = cy0 + cr;
      scx[k] = cx0 + c - cr * cw;
      const int64_t unit = ((int64_t)b * p.NQ + scy[k] * W + scx[k]) * p.NH + h;
      slx[k] = (float)loc[(unit * NP + pt) * 2];
      sly[k] = (float)loc[(unit * NP + pt) * 2 + 1];
      sa[k] = (float)attn[unit * NP + pt];
    }
    __syncthreads();  // the previous item's readers are done
    for (int i = tid; i < kOwnBins + 1; i += kOwnThreads) bin_at[i] = 0;
    __syncthreads();
    // Each near sample's corners inside the tile and the image: position and rank in the
    // position (integer LDS atomic), kept for the placement below.
    int pslot[kIter][4];
    float pwt[kIter][4];
#pragma unroll
    for (int k = 0; k < kIter; ++k) {
#pragma unroll
      for (int cn = 0; cn < 4; ++cn) pslot[k][cn] = -1;
      if (tid + k * kOwnThreads >= nsamp) continue;
      float him, wim;
      sample_coords<float>(slx[k], sly[k], H, W, him, wim);
      if (!(him > -1.f && wim > -1.f && him < (float)H && wim < (float)W)) continue;
      const float fh = floorf(him), fw = floorf(wim);
      const int hl = (int)fh, wl = (int)fw;
      if (!near_cell(hl, wl, scy[k], scx[k])) continue;
      const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
#pragma unroll
      for (int cn = 0; cn < 4; ++cn) {
        const int yy = hl + (cn >> 1), xx = wl + (cn & 1);
        const int ry = yy - y0, rx = xx - x0;
        if (yy < 0 || yy >= H || xx < 0 || xx >= W || (unsigned)ry >= (unsigned)kOwnT ||
            (unsigned)rx >= (unsigned)kOwnT)
          continue;
        const int bin = ry * kOwnT + rx;
        pslot[k][cn] = (bin << 16) | atomicAdd(&bin_at[bin], 1);
        pwt[k][cn] = ((cn >> 1) ? lh : hh) * ((cn & 1) ? lw : hw) * sa[k];
      }
    }
    __syncthreads();
    if (tid < kWave) {  // exclusive scan of the kOwnBins (= 64) counts by wave 0
      const int c = bin_at[tid];
      int incl = c;
#pragma unroll
      for (int d = 1; d < kWave; d <<= 1) {
        const int v = __shfl_up(incl, d, kWave);
        if (tid >= d) incl += v;
      }
      bin_at[tid] = incl - c;
      if (tid == kWave - 1) bin_at[kOwnBins] = incl;
    }
    __syncthreads();
    // Half-wave hw (0..15) owns positions [xb, xb + 4) of tile row r.
    constexpr int kHX = kOwnT / 2;
    const int hw = wave * 2 + half, r = hw >> 1, xb = (hw & 1) * kHX;
    float *gvr =
        p.gv + ((int64_t)b * p.S + (int64_t)(y0 + r) * W + x0 + xb) * (p.NH * D) + h * D + ch;
    const bool row_in = y0 + r < H;
    if (bin_at[kOwnBins] > kOwnCap) {
      // More pairs than the LDS list holds (inputs that crowd many samples into one
      // tile): zero the tile's rows (write mode), then every pair adds its weighted
      // grad_output row.
      if (!p.accumulate) {
#pragma unroll
        for (int x = 0; x < kHX; ++x)
          if (row_in && x0 + xb + x < W) gvr[(int64_t)x * (p.NH * D)] = 0.f;
      }
      __syncthreads();
      float *gvt = p.gv + ((int64_t)b * p.S + (int64_t)y0 * W + x0) * (p.NH * D) + h * D;
#pragma unroll
      for (int k = 0; k < kIter; ++k) {
#pragma unroll
        for (int cn = 0; cn < 4; ++cn)
          if (pslot[k][cn] >= 0) {
            const int bin = pslot[k][cn] >> 16;
            float *dst = gvt + ((int64_t)(bin / kOwnT) * W + bin % kOwnT) * (p.NH * D);
            const T *src = gout + b * p.go_sb + (int64_t)(scy[k] * W + scx[k]) * p.go_sq + h * p.go_sh;
            for (int e = 0; e < D; ++e) unsafeAtomicAdd(dst + e, pwt[k][cn] * (float)src[e * p.go_sc]);
          }
      }
      continue;
    }
#pragma unroll
    for (int k = 0; k < kIter; ++k) {
#pragma unroll
      for (int cn = 0; cn < 4; ++cn)
        if (pslot[k][cn] >= 0) {
          const int slot = bin_at[pslot[k][cn] >> 16] + (pslot[k][cn] & 0xffff);
          lq[slot] = scy[k] * W + scx[k];
          lw[slot] = pwt[k][cn];
        }
    }
    __syncthreads();
    // Lane ch of half-wave hw: channel ch; one position after the other, the sum of
    // weight x grad_output row (of the pair's query) over the position's pairs.
    const T *gob = gout + b * p.go_sb + h * p.go_sh + ch * p.go_sc;
    int bnd[kHX + 1];
#pragma unroll
    for (int x = 0; x <= kHX; ++x) bnd[x] = bin_at[r * kOwnT + xb + x];
    float old[kHX];  // accumulate mode: the positions' values, loaded before the sums
#pragma unroll
    for (int x = 0; x < kHX; ++x)
      old[x] = (p.accumulate && row_in && x0 + xb + x < W) ? gvr[(int64_t)x * (p.NH * D)] : 0.f;
#pragma unroll
    for (int x = 0; x < kHX; ++x) {
      float acc = 0.f;
      for (int k0 = bnd[x]; k0 < bnd[x + 1]; k0 += 8) {
        float w[8], v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = min(k0 + u, bnd[x + 1] - 1);
          w[u] = lw[k];
          v[u] = (float)gob[(int64_t)lq[k] * p.go_sq];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += (k0 + u < bnd[x + 1]) ? w[u] * v[u] : 0.f;
      }
      if (row_in && x0 + xb + x < W) gvr[(int64_t)x * (p.NH * D)] = old[x] + acc;
    }
  }
}

// ---------------------------------------------------------------------------
// grad_sampling_loc / grad_attn_weight for the owner path (one level, queries = cells,
// D = 32, P <= kOwnMaxP), plus the atomics of the samples the owner pass leaves out.
// G = D * sizeof(T) / 16 lanes own a (b, q, head) unit, lane li holding the VEC = 16 /
// sizeof(T) channels at li * VEC: the unit's P x 4 corner rows come in 16-byte pieces,
// all in flight together through the buffer path (corners outside the level or samples
// outside the window read zeros). The three outputs of a sample are fixed combinations
// of the corner dot products S_k = sum_c top_c * v_k,c:
//   grad_attn = sum_k w_k S_k,  grad_loc_x = W a (hh (S2 - S1) + lh (S4 - S3)),
//   grad_loc_y = H a (hw (S3 - S1) + lw (S4 - S2)),
// summed over the G lanes by a packed shuffle reduction.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kBlock) msda_grid_coord_kernel(
    const T *__restrict__ value, const T *__restrict__ loc, const T *__restrict__ attn,
    const T *__restrict__ grad_out, float *__restrict__ gv, T *__restrict__ grad_loc,
    T *__restrict__ grad_attn, BwdParams p) {
  constexpr int D = 32;
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int G = D / VEC;  // lanes per unit (8 fp32, 4 for 16-bit types)
  constexpr uint32_t kPast = 0x80000000u;
  // 32-bit unit indices and quotients from a float reciprocal corrected by one step (the
  // launch keeps units below 2^31 and every quotient below 2^22).
  auto qdiv = [](int a, int d) {
    int qq = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
    const int rr = a - qq * d;
    return qq + (rr >= d) - (rr < 0);
  };
  const int tid = blockIdx.x * kBlock + threadIdx.x;
  const int u_raw = tid / G;
  const bool live = u_raw < (int)p.units;
  const int unit = live ? u_raw : (int)p.units - 1;
  const int li = tid % G;
  const int bq = qdiv(unit, p.NH);
  const int h = unit - bq * p.NH;
  const int b = qdiv(bq, p.NQ);
  const int q = bq - b * p.NQ;
  const int NP = p.NP, NH = p.NH;
  const int H = (int)p.shapes[0], W = (int)p.shapes[1];
  const bool grid = grid_queries(p.shapes, p.lsi, p.NQ);
  const int qy = grid ? qdiv(q, W) : 0, qx = q - qy * W;
  const int64_t row = (int64_t)NH * D;
  // positions of the level inside the batch's value slice (the level's first position is
  // lsi[0]; corners at or past `avail` count as outside the level)
  const int64_t lsi0 = min(max(p.lsi[0], (int64_t)0), (int64_t)p.S);
  const int64_t avail = min((int64_t)H * W, (int64_t)p.S - lsi0);
  const T *vb = value + ((int64_t)b * p.S + lsi0) * row;
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vb, (uint32_t)(avail * row * sizeof(T)));
  const uint32_t lane_off = (uint32_t)((h * D + li * VEC) * sizeof(T));
  const T *go = grad_out + b * p.go_sb + (int64_t)q * p.go_sq + h * p.go_sh;
  float top[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) top[e] = (float)go[(li * VEC + e) * p.go_sc];
  float *gvb = gv + ((int64_t)b * p.S + lsi0) * row + h * D + li * VEC;
  const T *lp = loc + (int64_t)unit * NP * 2;
  const T *ap = attn + (int64_t)unit * NP;
  T *glp = grad_loc + (int64_t)unit * NP * 2;
  T *gap = grad_attn + (int64_t)unit * NP;

  // Geometry and corner loads of every point first.
  float wt[kOwnMaxP][4], lhs[kOwnMaxP], lws[kOwnMaxP], av[kOwnMaxP];
  int hls[kOwnMaxP], wls[kOwnMaxP];
  bool far[kOwnMaxP], okp[kOwnMaxP];
  Vec<T, VEC> cv[kOwnMaxP][4];
#pragma unroll
  for (int pt = 0; pt < kOwnMaxP; ++pt) {
    const int ps = pt < NP ? pt : 0;
    const float lx = (float)lp[2 * ps], ly = (float)lp[2 * ps + 1];
    av[pt] = (float)ap[ps];
    float him, wim;
    sample_coords<float>(lx, ly, H, W, him, wim);
    const bool ok = pt < NP && him > -1.f && wim > -1.f && him < (float)H && wim < (float)W;
    const float fh = ok ? floorf(him) : 0.f, fw = ok ? floorf(wim) : 0.f;
    const int hl = (int)fh, wl = (int)fw;
    const float lh = ok ? him - fh : 0.f, lw = ok ? wim - fw : 0.f;
    const float hh = 1.f - lh, hw = 1.f - lw;
    lhs[pt] = lh;
    lws[pt] = lw;
    hls[pt] = hl;
    wls[pt] = wl;
    okp[pt] = ok;
    far[pt] = ok && (!grid || !near_cell(hl, wl, qy, qx));
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int yy = hl + (k >> 1), xx = wl + (k & 1);
      const bool in = ok && yy >= 0 && yy < H && xx >= 0 && xx < W &&
                      (int64_t)yy * W + xx < avail;
      wt[pt][k] = in ? ((k >> 1) ? lh : hh) * ((k & 1) ? lw : hw) : 0.f;
      const uint32_t off = in ? (uint32_t)(((int64_t)yy * W + xx) * row * sizeof(T)) + lane_off : kPast;
      cv[pt][k] = buffer_load_vec<T, VEC>(rv, off);
    }
  }
#pragma unroll
  for (int pt = 0; pt < kOwnMaxP; ++pt) {
    if (pt < NP) {
    float s[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float acc = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc = fmaf(top[e], (float)cv[pt][k].v[e], acc);
      s[k] = acc;
    }
    // packed reduction of s[0..3] over the G lanes; lane 0 ends with all four sums
    const int hf = G >> 1, qt = G >> 2;
    const bool up = li & hf;
    float x = up ? s[2] : s[0], y = up ? s[3] : s[1];
    x += __shfl_xor(up ? s[0] : s[2], hf, kWave);
    y += __shfl_xor(up ? s[1] : s[3], hf, kWave);
    const bool up2 = li & qt;
    float v = up2 ? y : x;
    v += __shfl_xor(up2 ? x : y, qt, kWave);
    for (int st = qt >> 1; st >= 1; st >>= 1) v += __shfl_xor(v, st, kWave);
    const int base = (threadIdx.x & (kWave - 1)) & ~(G - 1);
    const float S1 = v, S2 = __shfl(v, base + qt, kWave);
    const float S3 = __shfl(v, base + hf, kWave), S4 = __shfl(v, base + hf + qt, kWave);
    if (live && li == 0) {  // a sample outside the window writes zeros
      const float lh = lhs[pt], lw = lws[pt], hh = 1.f - lh, hw = 1.f - lw, a = av[pt];
      const bool ok = okp[pt];
      glp[2 * pt] = (T)(ok ? (float)W * a * (hh * (S2 - S1) + lh * (S4 - S3)) : 0.f);
      glp[2 * pt + 1] = (T)(ok ? (float)H * a * (hw * (S3 - S1) + lw * (S4 - S2)) : 0.f);
      gap[pt] = (T)(ok ? wt[pt][0] * S1 + wt[pt][1] * S2 + wt[pt][2] * S3 + wt[pt][3] * S4 : 0.f);
    }
    if (live && far[pt]) {  // samples the owner pass does not take: atomics
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // every corner inside the map, weight 0 included (0 * a non-finite grad_output is
        // NaN in the reference's add, ms_deform_attn_kernels.cuh:445-480)
        const int yy = hls[pt] + (k >> 1), xx = wls[pt] + (k & 1);
        if (yy < 0 || yy >= H || xx < 0 || xx >= W || (int64_t)yy * W + xx >= avail) continue;
        float *dst = gvb + ((int64_t)yy * W + xx) * row;
        const float ta = wt[pt][k] * av[pt];
#pragma unroll
        for (int e = 0; e < VEC; ++e) unsafeAtomicAdd(dst + e, ta * top[e]);
      }
    }
    }
  }
}

// ---------------------------------------------------------------------------
// grad_value of the coarse levels (D = 32, fp32 accumulation) with one atomic per
// (position, channel) per workgroup instead of one per (sample, corner, channel): a
// persistent 8-wave workgroup takes kCoarseQ queries of one (batch, head) slice at a time,
//   1. stages their grad_output rows in LDS and counts every valid corner of their
//      coarse-level samples in its position (integer LDS atomic);
//   2. scans the counts, and a second visit of the samples stores the pairs
//      (query, bilinear weight x attention) in position order; the scanned counts give
//      each position's range, so a pair does not carry its position;
//   3. half-wave r streams an equal share of the pairs, summing weight x staged row, and
//      adds the sum to grad_value when the position changes (the position of its first
//      pair found by a binary search of the ranges).
// SCA's levels 2 and 3 (1825 positions) receive ~9 corner adds per position and slice
// from 256 queries, level 3 ~44: most of them collapse into one atomic. A workgroup whose
// pairs exceed the LDS list adds them one by one.
// ---------------------------------------------------------------------------
constexpr int kCoarseQ = 256;
constexpr int kCoarseThreads = 512;
constexpr int kCoarseCap = 16384;  // pairs kept in LDS (SCA: 256 queries x 2 levels x 8 x 4)
constexpr int kCoarseMaxSPU = 32;  // coarse samples per query the kernel takes (levels x points)
constexpr int kCoarseIter = kCoarseQ * kCoarseMaxSPU / kCoarseThreads;  // samples per thread

struct CoarseParams {
  const void *loc, *attn, *grad_out;
  float *gv;
  const int64_t *shapes, *lsi;
  int64_t go_sb, go_sq, go_sh, go_sc;
  int B, NH, NQ, NL, NP, S;
  int blocks_per_xcd;
};

template <typename T>
__global__ void __launch_bounds__(kCoarseThreads) msda_coarse_gv_kernel(const CoarseParams p) {
  constexpr int D = 32;
  __shared__ float tst[kCoarseQ * D];       // grad_output rows of the item's queries
  __shared__ int cnt[kCoarseBins + 1];      // counts, then each position's first pair
  __shared__ int cur[kCoarseBins];          // placement cursors
  __shared__ float lwt[kCoarseCap];         // pairs in position order: weight
  __shared__ unsigned short lq[kCoarseCap]; // and query in item
  __shared__ int wsum[kCoarseThreads / kWave];
  const int LC = coarse_first_level(p.shapes, p.lsi, p.NL, p.S);
  if (LC >= p.NL) return;  // uniform: no coarse level
  const int NLc = p.NL - LC;
  const int64_t base = p.lsi[LC];
  const int NB = (int)(p.lsi[p.NL - 1] + p.shapes[2 * (p.NL - 1)] * p.shapes[2 * p.NL - 1] - base);
  const int qchunks = (p.NQ + kCoarseQ - 1) / kCoarseQ;
  const int nitems = p.B * p.NH * qchunks;
  const int xcd = blockIdx.x & 7;
  const int per = (nitems + 7) / 8;
  const int i_end = min(nitems, (xcd + 1) * per);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int ch = tid & 31, hw = tid >> 5;  // half-wave index, 0..15
  const T *loc = static_cast<const T *>(p.loc);
  const T *attn = static_cast<const T *>(p.attn);
  const T *gout = static_cast<const T *>(p.grad_out);
  const int SPU = NLc * p.NP;  // coarse samples per query
  for (int item = xcd * per + (blockIdx.x >> 3); item < i_end; item += p.blocks_per_xcd) {
    const int qc = item % qchunks;
    const int bh = item / qchunks;
    const int h = bh % p.NH, b = bh / p.NH;
    const int q0 = qc * kCoarseQ;
    const int nq = min(kCoarseQ, p.NQ - q0);
    const int nsamp = nq * SPU;
    float *gvb = p.gv + ((int64_t)b * p.S + base) * (p.NH * D) + h * D;
    // The thread's coarse samples i = tid + k * kCoarseThreads: locations, weights and
    // level loaded once per item, all in flight together, for both visits below.
    float slx[kCoarseIter], sly[kCoarseIter], sa[kCoarseIter];
    int sl[kCoarseIter];
#pragma unroll
    for (int k = 0; k < kCoarseIter; ++k) {
      const int i = min(tid + k * kCoarseThreads, nsamp - 1);
      const int u = i / SPU, r = i - u * SPU;
      const int lv = r / p.NP, pt = r - lv * p.NP;
      sl[k] = LC + lv;
      const int64_t unit = ((int64_t)b * p.NQ + q0 + u) * p.NH + h;
      const int64_t si = (unit * p.NL + sl[k]) * p.NP + pt;
      slx[k] = (float)loc[si * 2];
      sly[k] = (float)loc[si * 2 + 1];
      sa[k] = (float)attn[si];
    }
    // Calls fn(position, query in item, weight) for every valid corner of the thread's
    // k-th coarse sample.
    auto visit = [&](int k, auto &&fn) __attribute__((always_inline)) {
      const int i = tid + k * kCoarseThreads;
      if (i >= nsamp) return;
      const int u = i / SPU;
      const int l = sl[k];
      const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
      float him, wim;
      sample_coords<float>(slx[k], sly[k], Hl, Wl, him, wim);
      if (!(him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl)) return;
      const float fh = floorf(him), fw = floorf(wim);
      const int hl = (int)fh, wl = (int)fw;
      const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hwt = 1.f - lw;
      const int lbase = (int)(p.lsi[l] - base);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int yy = hl + (c >> 1), xx = wl + (c & 1);
        if (yy < 0 || yy >= Hl || xx < 0 || xx >= Wl) continue;
        fn(lbase + yy * Wl + xx, u, ((c >> 1) ? lh : hh) * ((c & 1) ? lw : hwt) * sa[k]);
      }
    };
    __syncthreads();  // the previous item's readers are done
    for (int i = tid; i < nq * D; i += kCoarseThreads) {
      const int u = i / D, c = i - u * D;
      tst[i] = (float)gout[b * p.go_sb + (int64_t)(q0 + u) * p.go_sq + h * p.go_sh + c * p.go_sc];
    }
    for (int i = tid; i <= NB; i += kCoarseThreads) cnt[i] = 0;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kCoarseIter; ++k) visit(k, [&](int bin, int, float) { atomicAdd(&cnt[bin], 1); });
    __syncthreads();
    {  // exclusive scan of the NB counts: thread tid owns [tid*E, tid*E + E)
      const int E = (NB + kCoarseThreads - 1) / kCoarseThreads;
      const int e0 = min(tid * E, NB), e1 = min(e0 + E, NB);
      int local = 0;
      for (int e = e0; e < e1; ++e) local += cnt[e];
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
        const int c = cnt[e];
        cnt[e] = run;
        cur[e] = run;
        run += c;
      }
      if (tid == kCoarseThreads - 1) {
        int tot = 0;
        for (int w2 = 0; w2 < kCoarseThreads / kWave; ++w2) tot += wsum[w2];
        cnt[NB] = tot;
      }
    }
    __syncthreads();
    const int total = cnt[NB];
    if (total > kCoarseCap) {
      // More pairs than the LDS list holds: every pair adds its weighted row directly.
#pragma unroll
      for (int k = 0; k < kCoarseIter; ++k)
        visit(k, [&](int bin, int u, float w) {
          for (int c = 0; c < D; ++c) unsafeAtomicAdd(gvb + (int64_t)bin * (p.NH * D) + c, w * tst[u * D + c]);
        });
      continue;
    }
#pragma unroll
    for (int k = 0; k < kCoarseIter; ++k)
      visit(k, [&](int bin, int u, float w) {
        const int slot = atomicAdd(&cur[bin], 1);
        lwt[slot] = w;
        lq[slot] = (unsigned short)u;
      });
    __syncthreads();
    // Half-wave hw streams pairs [total * hw / 16, total * (hw + 1) / 16); lane ch holds
    // channel ch; a position cut by two half-waves is added in two parts.
    const int lo = total * hw / (kCoarseThreads / 32), hi = total * (hw + 1) / (kCoarseThreads / 32);
    if (lo < hi) {
      // the position holding pair lo: the last one whose range starts at or before lo
      // (an empty position's successor starts where it does, so the last one is not empty)
      int bin = 0;
      for (int st = kCoarseBins / 2; st > 0; st >>= 1)
        if (bin + st < NB && cnt[bin + st] <= lo) bin += st;
      int next = cnt[bin + 1];  // first pair of the following position
      float acc = 0.f;
      for (int k0 = lo; k0 < hi; k0 += 8) {
        float w[8], v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = min(k0 + u, hi - 1);
          w[u] = lwt[k];
          v[u] = tst[lq[k] * D + ch];
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int k = k0 + u;
          if (k < hi) {
            if (k >= next) {  // pair k starts a later position (k < total ends the walk)
              unsafeAtomicAdd(gvb + (int64_t)bin * (p.NH * D) + ch, acc);
              acc = 0.f;
              do {
                ++bin;
                next = cnt[bin + 1];
              } while (next <= k);
            }
            acc += w[u] * v[u];
          }
        }
      }
      unsafeAtomicAdd(gvb + (int64_t)bin * (p.NH * D) + ch, acc);
    }
  }
}

// ---------------------------------------------------------------------------
// msda_col2im_kernel for D = 32 and fp32 accumulation (the BEVFormer shapes): 32 lanes per
// (b, q, head) unit, lane c on channel c, two units per wave. Same per-sample arithmetic;
// 32-bit offsets (one batch of value under 2 GiB, checked at launch), quotients by the
// runtime sizes from a reciprocal with one correction step, corner loads through the
// buffer path with out-of-level corners reading zeros (no branches around the loads), and
// the three channel sums of a sample reduced in 8 shuffles (each quarter of the 32 lanes
// ends up holding one of them) instead of 15. The kernel was VALU-bound beside its
// atomics: ~5,900 VALU instructions per wave at SCA.
// ---------------------------------------------------------------------------
template <typename T>
__global__ void __launch_bounds__(kBlock) msda_col2im_d32_kernel(
    const T *__restrict__ value, const T *__restrict__ loc, const T *__restrict__ attn,
    const T *__restrict__ grad_out, float *__restrict__ grad_value, T *__restrict__ grad_loc,
    T *__restrict__ grad_attn, BwdParams p) {
  constexpr int D = 32;
  constexpr uint32_t kPast = 0x80000000u;
  auto qdiv = [](int a, int d) {
    int qq = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
    const int rr = a - qq * d;
    return qq + (rr >= d) - (rr < 0);
  };
  const int tid = blockIdx.x * kBlock + threadIdx.x;
  const int u_raw = tid >> 5;
  const bool live = u_raw < (int)p.units;
  const int unit = live ? u_raw : (int)p.units - 1;
  const int lane = tid & 31;
  const int bq = qdiv(unit, p.NH);
  const int h = unit - bq * p.NH;
  const int b = qdiv(bq, p.NQ);
  const int q = bq - b * p.NQ;
  const int NS = p.NL * p.NP;
  const int row = p.NH * D;  // elements per spatial position
  const float top = live ? (float)grad_out[b * p.go_sb + (int64_t)q * p.go_sq + h * p.go_sh +
                                           lane * p.go_sc]
                         : 0.f;
  const T *vb = value + (int64_t)b * p.S * row + h * D;
  float *gvb = grad_value + (int64_t)b * p.S * row + h * D;
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(vb, (uint32_t)(((int64_t)p.S * row - h * D) * sizeof(T)));
  const T *lp = loc + (int64_t)unit * NS * 2;
  const T *ap = attn + (int64_t)unit * NS;
  T *glp = grad_loc + (int64_t)unit * NS * 2;
  T *gap = grad_attn + (int64_t)unit * NS;
  const int LC = p.coarse ? coarse_first_level(p.shapes, p.lsi, p.NL, p.S) : p.NL;
  const uint32_t lane_b = (uint32_t)(lane * sizeof(T));
  for (int l = 0; l < p.NL; ++l) {
    const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
    const int base = (int)p.lsi[l];
    const bool add = live && l < LC;  // coarse levels: msda_coarse_gv_kernel
    for (int pt = 0; pt < p.NP; ++pt) {
      const int s = l * p.NP + pt;
      const float lx = (float)lp[2 * s], ly = (float)lp[2 * s + 1], a = (float)ap[s];
      float him, wim;
      sample_coords<float>(lx, ly, Hl, Wl, him, wim);
      float gh = 0.f, gw = 0.f, ga = 0.f;
      if (him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl) {
        const float fh = floorf(him), fw = floorf(wim);
        const int hl = (int)fh, wl = (int)fw;
        const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
        const float w1 = hh * hw, w2 = hh * lw, w3 = lh * hw, w4 = lh * lw;
        const bool c1 = hl >= 0 && wl >= 0, c2 = hl >= 0 && wl + 1 <= Wl - 1;
        const bool c3 = hl + 1 <= Hl - 1 && wl >= 0;
        const bool c4 = hl + 1 <= Hl - 1 && wl + 1 <= Wl - 1;
        const int e1 = (base + hl * Wl + wl) * row, e2 = e1 + row;
        const int e3 = e1 + Wl * row, e4 = e3 + row;
        const uint32_t eb = (uint32_t)sizeof(T);
        const float v1 = (float)buffer_load_one<T>(rv, c1 ? (uint32_t)e1 * eb + lane_b : kPast);
        const float v2 = (float)buffer_load_one<T>(rv, c2 ? (uint32_t)e2 * eb + lane_b : kPast);
        const float v3 = (float)buffer_load_one<T>(rv, c3 ? (uint32_t)e3 * eb + lane_b : kPast);
        const float v4 = (float)buffer_load_one<T>(rv, c4 ? (uint32_t)e4 * eb + lane_b : kPast);
        const float ta = top * a;
        if (add) {
          if (c1) unsafeAtomicAdd(gvb + e1 + lane, w1 * ta);
          if (c2) unsafeAtomicAdd(gvb + e2 + lane, w2 * ta);
          if (c3) unsafeAtomicAdd(gvb + e3 + lane, w3 * ta);
          if (c4) unsafeAtomicAdd(gvb + e4 + lane, w4 * ta);
        }
        gh = ta * (hw * (v3 - v1) + lw * (v4 - v2)) * (float)Hl;
        gw = ta * (hh * (v2 - v1) + lh * (v4 - v3)) * (float)Wl;
        ga = top * (w1 * v1 + w2 * v2 + w3 * v3 + w4 * v4);
      }
      // lanes 0-15 keep (gh, gw), 16-31 keep ga; then each quarter keeps one sum
      const bool up = lane & 16;
      float k1 = up ? ga : gh, k2 = up ? 0.f : gw;
      k1 += __shfl_xor(up ? gh : ga, 16, kWave);
      k2 += __shfl_xor(up ? gw : 0.f, 16, kWave);
      const bool up2 = lane & 8;
      float v = up2 ? k2 : k1;
      v += __shfl_xor(up2 ? k1 : k2, 8, kWave);
      v += __shfl_xor(v, 4, kWave);
      v += __shfl_xor(v, 2, kWave);
      v += __shfl_xor(v, 1, kWave);
      const int base_lane = (threadIdx.x & (kWave - 1)) & ~31;
      const float sgw = __shfl(v, base_lane + 8, kWave), sga = __shfl(v, base_lane + 16, kWave);
      if (live && lane == 0) {
        glp[2 * s] = (T)sgw;
        glp[2 * s + 1] = (T)v;
        gap[s] = (T)sga;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Sorted grad_value path (D = 32, fp32 accumulation, every level). The fp32 atomics of
// msda_col2im_d32_kernel add one 128-byte row per valid corner (30.7 M rows for the fine
// levels of SCA), at the L2's atomic line rate. Here the corner adds are bucketed by
// position instead, and every bucket of kBkPos consecutive positions of a (batch, head)
// slice is summed by one workgroup that owns those grad_value rows. The unit of the sort
// is a record: the two corners of one image row of a sample (x0 and x0 + 1, positions p
// and p + 1) share the sample's grad_output row, so a record carries the first valid
// position of the pair and two weights, for that position and for the next one (0 when
// only one corner of the pair is valid); a sample gives at most two records.
//   1. msda_bkt_count_kernel: the records of every sample counted per bucket (LDS
//      histogram per block, one global add per bucket and block);
//   2. msda_bkt_scan_kernel: bucket offsets and placement cursors, and the chunks of the
//      non-empty buckets listed per XCD (slice % 8, or bucket % 8 with fewer than 8
//      slices) with 16-byte headers;
//   3. msda_bkt_place_kernel: the records again, staged in LDS in bucket order, each
//      bucket's range reserved once per block, then written as contiguous runs of
//      (weight, next weight) pairs and (query << kBkShift | position in bucket) words;
//   4. msda_bkt_acc_kernel: per chunk of at most kAccChunk records of one bucket, a
//      counting sort by position in LDS; each group of 16-byte lanes (8 for fp32, 4 for
//      16-bit types: one grad_output row) takes whole positions (about 1/64 or 1/128 of
//      the chunk's records), sums weight x grad_output row into two register sums
//      (position, next position) and stores each position's sum to an LDS accumulator
//      once; the next-position sum of a group's last position is added after a barrier.
//      The accumulator has one row more than the bucket (the next bucket's first position,
//      reached by records at the bucket's last position). It is added to grad_value at the
//      end: with plain read-modify-writes when the bucket is one chunk (no other workgroup
//      writes these rows), else with atomics; the first row and the extra row, which the
//      neighbouring buckets also reach, always with atomics.
// grad_sampling_loc / grad_attn_weight come from msda_coord_kernel (no atomics).
// Corner set and weights are those of the reference (ms_deform_attn_kernels.cuh:427-490):
// the same in-window test and per-corner bounds, weight = bilinear weight x attention.
// ---------------------------------------------------------------------------
constexpr int kBkShift = 8;
constexpr int kBkPos = 1 << kBkShift;      // positions per bucket
constexpr int kBkMaxPerSlice = 1024;       // buckets per slice (spatial_size <= 256 Ki)
constexpr int kBkThreads = 256;
constexpr int kChunkSamples = 1024;        // samples per count / place chunk
constexpr int kChunkRecs = 2 * kChunkSamples;  // records a place block stages
constexpr int kAccThreads = 512;
constexpr int kAccChunk = 3584;            // records per accumulate chunk (79 KB LDS; 2 blocks per CU)
constexpr int kAccPerThread = kAccChunk / kAccThreads;
constexpr int kAccPiece = 2;               // chunks of one bucket a workgroup sums in turn

struct BktParams {
  const void *loc, *attn, *grad_out;
  const int64_t *shapes, *lsi;
  float *gv;
  int *count;       // [nbk] records per bucket
  int *cursor;      // [nbk] next free slot (offsets after the scan)
  int *offset;      // [nbk + 1]
  int *nitems;      // [8] pieces per XCD list, then [8] work-queue counters
  int4 *items;      // [8][item_cap] (bucket, first record, records, 1 if the bucket is one piece)
  float2 *rw;       // [capacity] record weights: (position, next position)
  uint32_t *rq;     // [capacity] query << kBkShift | position in bucket
  int64_t go_sb, go_sq, go_sh, go_sc;
  uint32_t go_rows_bytes;  // bytes from row (b, 0, h, 0) past row (b, NQ - 1, h, 31)
  int B, NH, NQ, NL, NP, S, NBS, nbk, item_cap, qpb;
  int by_bucket;    // fewer than 8 slices: buckets go to XCD bucket % 8, else slice % 8
  int blocks_per_xcd;
  int cblk8;        // count / place chunks per XCD
  int pblk;         // count / place blocks per XCD (persistent)
  float *zero;      // 16-bit types: the fp32 grad_value workspace, cleared by the count
  int64_t nzero4;   //   kernel (float4 groups; 0: nothing to clear)
};

// a / d for 0 <= a < 2^24 and 0 < d: a reciprocal estimate and one correction step
__device__ __forceinline__ int fast_div(int a, int d) {
  int q = (int)((float)a * __builtin_amdgcn_rcpf((float)d));
  const int r = a - q * d;
  return q + (r >= d) - (r < 0);
}

// Count and place work in chunks of qpb queries of one (batch, head) slice (at most
// kChunkSamples samples). The chunks are numbered slice by slice and XCD x (block index
// % 8) takes the x-th eighth of them, so the blocks of one XCD work on one or two slices at
// a time and a bucket's records are written through one L2. The blocks are persistent:
// block r of an XCD takes its chunks r, r + pblk, ..., and the next chunk's locations and
// attention weights are loaded while the current one is processed.
constexpr int kBkSPT = kChunkSamples / kBkThreads;  // samples of a chunk per thread

template <typename T>
struct ChunkSamples {
  Vec<T, 2> xy[kBkSPT];
  T a[kBkSPT];
};

__device__ __forceinline__ void bkt_chunk(const BktParams &p, int lb, int &slice, int &q0,
                                          int &nq) {
  const int qchunks = (p.NQ + p.qpb - 1) / p.qpb;
  slice = lb / qchunks;
  q0 = (lb - slice * qchunks) * p.qpb;
  nq = min(p.qpb, p.NQ - q0);
}

// This XCD's chunk range [lb0, lb1).
__device__ __forceinline__ void bkt_range(const BktParams &p, int &lb0, int &lb1) {
  const int total = p.B * p.NH * ((p.NQ + p.qpb - 1) / p.qpb);
  lb0 = min((int)(blockIdx.x & 7) * p.cblk8, total);
  lb1 = min(lb0 + p.cblk8, total);
}

// Sample i = threadIdx.x + j * kBkThreads of chunk lb (a thread past the chunk's samples
// reads the last one again).
template <typename T>
__device__ __forceinline__ void load_chunk(const BktParams &p, int lb, ChunkSamples<T> &cs) {
  int slice, q0, nq;
  bkt_chunk(p, lb, slice, q0, nq);
  const int b = slice / p.NH, h = slice - b * p.NH, NS = p.NL * p.NP;
  const T *loc = static_cast<const T *>(p.loc);
  const T *attn = static_cast<const T *>(p.attn);
#pragma unroll
  for (int j = 0; j < kBkSPT; ++j) {
    const int i = min((int)threadIdx.x + j * kBkThreads, nq * NS - 1);
    const int u = fast_div(i, NS), r = i - u * NS;
    const int64_t si = (((int64_t)b * p.NQ + q0 + u) * p.NH + h) * NS + r;
    cs.xy[j] = *reinterpret_cast<const Vec<T, 2> *>(loc + si * 2);
    cs.a[j] = attn[si];
  }
}

// The four corners of a sample of level l at location xy with attention weight a:
// position (-1 for an invalid corner or a sample outside the window) and weight.
// Positions outside [0, S) (inconsistent metadata) count as invalid.
template <typename T>
__device__ __forceinline__ void sample_corners(const BktParams &p, int l, const Vec<T, 2> &xy,
                                               T at, int (&pos)[4], float (&wt)[4]) {
  const float lx = (float)xy.v[0], ly = (float)xy.v[1], a = (float)at;
  const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
  float him, wim;
  sample_coords<float>(lx, ly, Hl, Wl, him, wim);
  const bool in = him > -1.f && wim > -1.f && him < (float)Hl && wim < (float)Wl;
  const float fh = floorf(him), fw = floorf(wim);
  const int hl = (int)fh, wl = (int)fw;
  const float lh = him - fh, lw = wim - fw, hh = 1.f - lh, hw = 1.f - lw;
  const int64_t base = p.lsi[l];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int yy = hl + (c >> 1), xx = wl + (c & 1);
    const int64_t ps = base + (int64_t)yy * Wl + xx;
    const bool ok = in && yy >= 0 && yy < Hl && xx >= 0 && xx < Wl && ps >= 0 && ps < p.S;
    pos[c] = ok ? (int)ps : -1;
    wt[c] = ((c >> 1) ? lh : hh) * ((c & 1) ? lw : hw) * a;
  }
}

// The two records of a sample (r = 0: corners 0 and 1, image row y0; r = 1: corners 2 and
// 3, row y0 + 1). Both corners valid: position of the left one, weights (left, right);
// one valid: its position, weights (its weight, 0); none: position -1. The right corner of
// a row is the position after the left one.
template <typename T>
__device__ __forceinline__ void sample_records(const BktParams &p, int l, const Vec<T, 2> &xy,
                                               T at, int (&rp)[2], float2 (&rw)[2]) {
  int pos[4];
  float wt[4];
  sample_corners<T>(p, l, xy, at, pos, wt);
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int a = pos[2 * r], b = pos[2 * r + 1];
    rp[r] = a >= 0 ? a : b;
    rw[r] = a >= 0 ? make_float2(wt[2 * r], b >= 0 ? wt[2 * r + 1] : 0.f)
                   : make_float2(wt[2 * r + 1], 0.f);
  }
}

template <typename T>
__global__ void __launch_bounds__(kBkThreads) msda_bkt_count_kernel(const BktParams p) {
  __shared__ int lcnt[kBkMaxPerSlice];
  const int NS = p.NL * p.NP;
  int lb0, lb1;
  bkt_range(p, lb0, lb1);
  ChunkSamples<T> cs;
  int lb = lb0 + (int)(blockIdx.x >> 3);
  if (lb < lb1) load_chunk<T>(p, lb, cs);
  // the fp32 workspace of 16-bit types, cleared here (the accumulate kernel adds to it
  // after this kernel): the block's share in 16-byte stores, a few per thread and chunk
  // so that they stream out while the blocks compute, the rest after the last chunk
  const int64_t zper = (p.nzero4 + gridDim.x - 1) / gridDim.x;
  const int64_t z0 = (int64_t)blockIdx.x * zper, z1 = min(z0 + zper, p.nzero4);
  const int nit = lb < lb1 ? (lb1 - 1 - lb) / p.pblk + 1 : 1;  // this block's chunks
  const int64_t zstep = ((z1 - z0 + kBkThreads - 1) / kBkThreads + nit - 1) / nit * kBkThreads;
  int64_t zi = z0;
  auto clear_some = [&](int64_t upto) __attribute__((always_inline)) {
    for (int64_t i = zi + threadIdx.x; i < upto; i += kBkThreads)
      reinterpret_cast<float4 *>(p.zero)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    zi = upto;
  };
  for (; lb < lb1; lb += p.pblk) {
    if (zi < z1) clear_some(min(zi + zstep, z1));
    int slice, q0, nq;
    bkt_chunk(p, lb, slice, q0, nq);
    int pos[kBkSPT][2];
#pragma unroll
    for (int j = 0; j < kBkSPT; ++j) {
      const int i = threadIdx.x + j * kBkThreads;
      const int l = fast_div(i - fast_div(i, NS) * NS, p.NP);
      float2 wt[2];
      sample_records<T>(p, i < nq * NS ? l : 0, cs.xy[j], cs.a[j], pos[j], wt);
      if (i >= nq * NS) pos[j][0] = pos[j][1] = -1;
    }
    if (lb + p.pblk < lb1) load_chunk<T>(p, lb + p.pblk, cs);  // in flight during this chunk
    __syncthreads();  // the previous chunk's flush is done
    for (int k = threadIdx.x; k < p.NBS; k += kBkThreads) lcnt[k] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kBkSPT; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (pos[j][r] >= 0) atomicAdd(&lcnt[pos[j][r] >> kBkShift], 1);
    __syncthreads();
    for (int k = threadIdx.x; k < p.NBS; k += kBkThreads)
      if (lcnt[k] > 0) atomicAdd(&p.count[slice * p.NBS + k], lcnt[k]);
  }
  if (zi < z1) clear_some(z1);
}

// Block x (of 8): exclusive scan of the bucket counts (block 0 stores offset and cursor),
// then list x: the buckets of XCD x cut into pieces of at most kAccPiece chunks of
// kAccChunk records, pieces of several chunks first (the accumulate workgroups take them
// from a queue, so the long ones start early). Thread t owns a contiguous run of buckets:
// one pass to count, one block scan of the run totals, one pass to write.
__global__ void __launch_bounds__(1024) msda_bkt_scan_kernel(const BktParams p) {
  constexpr int kPieceRecs = kAccPiece * kAccChunk;
  __shared__ int wsum[3][16];
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int x = blockIdx.x;
  const int E = (p.nbk + 1023) / 1024;
  const int k0 = min(tid * E, p.nbk), k1 = min(k0 + E, p.nbk);
  auto mine = [&](int k) __attribute__((always_inline)) {
    return ((p.by_bucket ? k : k / p.NBS) & 7) == x;
  };
  // pieces of a bucket of c records: full pieces, then the rest; "long" = several chunks
  auto pieces = [&](int c, int &nlong, int &nshort) __attribute__((always_inline)) {
    const int full = c / kPieceRecs, rest = c - full * kPieceRecs;
    nlong = full + (rest > kAccChunk);
    nshort = rest > 0 && rest <= kAccChunk;
  };
  int v[3] = {0, 0, 0};  // records, long pieces, short pieces
  for (int k = k0; k < k1; k += 4) {
    int c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = k + j < k1 ? p.count[k + j] : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[0] += c[j];
      if (k + j < k1 && mine(k + j)) {
        int nl, ns;
        pieces(c[j], nl, ns);
        v[1] += nl;
        v[2] += ns;
      }
    }
  }
  int incl[3] = {v[0], v[1], v[2]};
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      const int t = __shfl_up(incl[r], d, kWave);
      if (lane >= d) incl[r] += t;
    }
  }
  if (lane == kWave - 1) {
#pragma unroll
    for (int r = 0; r < 3; ++r) wsum[r][wave] = incl[r];
  }
  __syncthreads();
  int run[3], total[3];
#pragma unroll
  for (int r = 0; r < 3; ++r) {
    run[r] = incl[r] - v[r];
    total[r] = 0;
    for (int w = 0; w < 16; ++w) {
      if (w < wave) run[r] += wsum[r][w];
      total[r] += wsum[r][w];
    }
  }
  int rl = run[1], rs = total[1] + run[2];  // list slots of this run's long / short pieces
  int4 *list = p.items + (int64_t)x * p.item_cap;
  int off = run[0];
  for (int k = k0; k < k1; ++k) {
    const int c = p.count[k];
    if (x == 0) {
      p.offset[k] = off;
      p.cursor[k] = off;
    }
    if (mine(k)) {
      const int whole = c <= kPieceRecs;
      for (int f = 0; f < c; f += kPieceRecs) {
        const int n = min(kPieceRecs, c - f);
        int &slot = n > kAccChunk ? rl : rs;
        if (slot < p.item_cap) list[slot] = make_int4(k, off + f, n, whole);
        ++slot;
      }
    }
    off += c;
  }
  if (tid == 0) {
    if (x == 0) p.offset[p.nbk] = total[0];
    p.nitems[x] = min(total[1] + total[2], p.item_cap);
    p.nitems[8 + x] = 0;  // the accumulate kernel's queue
  }
}

// Same chunks as the count kernel (qpb * L * P <= kChunkSamples samples): per chunk, the
// records of the thread's samples (kept in registers), counted per bucket, staged in LDS in
// bucket order, each bucket's range reserved once, then written as contiguous runs.
template <typename T>
__global__ void __launch_bounds__(kBkThreads) msda_bkt_place_kernel(const BktParams p) {
  constexpr int SPT = kBkSPT;
  __shared__ int lcnt[kBkMaxPerSlice];   // counts, then staging cursors
  __shared__ int gofs[kBkMaxPerSlice];   // global slot - staged index of each bucket's records
  __shared__ float2 sw[kChunkRecs];
  __shared__ uint32_t sq[kChunkRecs];
  __shared__ unsigned short sb[kChunkRecs];
  __shared__ int wsum[kBkThreads / kWave];
  const int NS = p.NL * p.NP;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  int lb0, lb1;
  bkt_range(p, lb0, lb1);
  ChunkSamples<T> cs;
  int lb = lb0 + (int)(blockIdx.x >> 3);
  if (lb < lb1) load_chunk<T>(p, lb, cs);
  for (; lb < lb1; lb += p.pblk) {
    int slice, q0, nq;
    bkt_chunk(p, lb, slice, q0, nq);
    int rpos[SPT][2];
    float2 rwt[SPT][2];
    uint32_t rq[SPT];
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const int i = tid + j * kBkThreads;
      const int u = fast_div(i, NS), l = fast_div(i - u * NS, p.NP);
      sample_records<T>(p, i < nq * NS ? l : 0, cs.xy[j], cs.a[j], rpos[j], rwt[j]);
      rq[j] = (uint32_t)(q0 + u) << kBkShift;
      if (i >= nq * NS) rpos[j][0] = rpos[j][1] = -1;
    }
    if (lb + p.pblk < lb1) load_chunk<T>(p, lb + p.pblk, cs);  // in flight during this chunk
    __syncthreads();  // the previous chunk's writers are done with the LDS
    for (int k = tid; k < p.NBS; k += kBkThreads) lcnt[k] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SPT; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (rpos[j][r] >= 0) atomicAdd(&lcnt[rpos[j][r] >> kBkShift], 1);
    __syncthreads();
    // exclusive scan of the NBS counts: thread tid owns [tid*E, tid*E + E), E <= 4; each
    // bucket's global range is reserved here, and the atomics' results are first used
    // after the staging below, which runs while they return
    constexpr int kMaxE = kBkMaxPerSlice / kBkThreads;
    static_assert(kMaxE * kBkThreads == kBkMaxPerSlice, "bucket runs per thread");
    const int E = (p.NBS + kBkThreads - 1) / kBkThreads;
    const int e0 = min(tid * E, p.NBS), e1 = min(e0 + E, p.NBS);
    int gres[kMaxE], gstart[kMaxE];
    {
      int local = 0;
      for (int e = e0; e < e1; ++e) local += lcnt[e];
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
#pragma unroll
      for (int j = 0; j < kMaxE; ++j) {
        const int e = e0 + j;
        gres[j] = 0;
        gstart[j] = run;
        if (e < e1) {
          const int c = lcnt[e];
          if (c > 0) gres[j] = atomicAdd(&p.cursor[slice * p.NBS + e], c);
          lcnt[e] = run;
          run += c;
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < SPT; ++j)
#pragma unroll
      for (int r = 0; r < 2; ++r)
        if (rpos[j][r] >= 0) {
          const int k = rpos[j][r] >> kBkShift;
          const int slot = atomicAdd(&lcnt[k], 1);
          sw[slot] = rwt[j][r];
          sq[slot] = rq[j] | (uint32_t)(rpos[j][r] & (kBkPos - 1));
          sb[slot] = (unsigned short)k;
        }
#pragma unroll
    for (int j = 0; j < kMaxE; ++j)
      if (e0 + j < e1) gofs[e0 + j] = gres[j] - gstart[j];
    __syncthreads();
    const int total = lcnt[p.NBS - 1];  // the last bucket's cursor ends at the staged total
    for (int i = tid; i < total; i += kBkThreads) {
      const int dst = gofs[sb[i]] + i;
      p.rw[dst] = sw[i];
      p.rq[dst] = sq[i];
    }
  }
}

// Persistent: the workgroups of XCD x take the pieces of list x from a queue (one atomic
// per piece, fetched one piece ahead). A piece is up to kAccPiece chunks of one bucket,
// summed one after the other into the LDS accumulator; its rows are added to grad_value
// once: with plain read-modify-writes when the piece is the whole bucket (no other
// workgroup writes those rows), else with atomics. The bucket's first row and the row
// after the bucket are also reached by the neighbouring buckets' records (and the pieces
// that sum them), so they always take atomics.
template <typename T>
__global__ void __launch_bounds__(kAccThreads, 4) msda_bkt_acc_kernel(const BktParams p) {
  // a group of LPC lanes reads one 128-byte (fp32) or 64-byte (16-bit) grad_output row,
  // 16 bytes per lane
  constexpr int D = 32, VEC = 16 / (int)sizeof(T), LPC = D / VEC;
  constexpr int NGR = kAccThreads / LPC;
  constexpr int BT = VEC == 4 ? 4 : 3;      // records per batch of a group (no spills)
  __shared__ float accs[(kBkPos + 1) * D];  // the piece's sums per position (+ the next bucket's first)
  __shared__ int cnt[kBkPos + 1];           // counts, then each position's first record
  __shared__ int cur[kBkPos];
  __shared__ float2 lw[kAccChunk];
  __shared__ uint32_t lq[kAccChunk];
  __shared__ int pcut[NGR + 1];             // first position of each group
  __shared__ int wsum[kAccThreads / kWave];
  __shared__ unsigned char touched[kBkPos + 1];  // rows the piece has added to so far
  __shared__ int s_next;
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
  const int cl = tid % LPC, gi = tid / LPC;
  const int xcd = blockIdx.x & 7;
  const int n_items = p.nitems[xcd];
  int *queue = p.nitems + 8 + xcd;
  const int4 *items = p.items + (int64_t)xcd * p.item_cap;
  const T *gout = static_cast<const T *>(p.grad_out);
  // the records of a chunk, kAccPerThread per thread (streamed once: non-temporal loads
  // keep the grad_output rows in L2)
  float2 rw[kAccPerThread];
  uint32_t rq[kAccPerThread];
  auto load_records = [&](int from, int n) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kAccPerThread; ++j) {
      const int i = min(tid + j * kAccThreads, n - 1);
      typedef float f2v __attribute__((ext_vector_type(2)));
      const f2v w = __builtin_nontemporal_load(reinterpret_cast<const f2v *>(p.rw + from + i));
      rw[j] = make_float2(w.x, w.y);
      rq[j] = __builtin_nontemporal_load(p.rq + from + i);
    }
  };
  // records at position pp of the current chunk (pp <= kBkPos; the extra row has none)
  auto has = [&](int pp) __attribute__((always_inline)) {
    return pp < kBkPos && cnt[pp + 1] > cnt[pp];
  };
  if (tid == 0) s_next = atomicAdd(queue, 1);
  __syncthreads();
  // the piece index is uniform: kept in a scalar register, so the piece header and every
  // address and buffer descriptor derived from it are scalar too
  int m = __builtin_amdgcn_readfirstlane(s_next);
  while (m < n_items) {
    const int4 it = items[m];  // (bucket, first record, records, whole bucket)
    __syncthreads();  // s_next is read; the previous piece's readers of the LDS are done
    if (tid == 0) s_next = atomicAdd(queue, 1);  // the next piece, fetched during this one
    const int k = it.x, first = it.y, np_ = it.z;
    const bool whole = it.w != 0;
    const bool multi = np_ > kAccChunk;  // several chunks: sums added up in LDS
    const int slice = k / p.NBS, kb = k - slice * p.NBS;
    const int b = slice / p.NH, h = slice - b * p.NH;
    // grad_output rows of (b, ., h) through a buffer over the batch's rows (32-bit offsets)
    const T *gob = gout + b * p.go_sb + h * p.go_sh;
    const __amdgpu_buffer_rsrc_t gr = make_rsrc(gob, p.go_rows_bytes);
    const uint32_t go_q_bytes = (uint32_t)(p.go_sq * (int64_t)sizeof(T));
    const uint32_t ch_bytes = (uint32_t)(cl * VEC * sizeof(T));  // channels are contiguous
    if (multi) {
      for (int i = tid; i < (kBkPos + 1) * D / 4; i += kAccThreads)
        reinterpret_cast<float4 *>(accs)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int i = tid; i <= kBkPos; i += kAccThreads) touched[i] = 0;
    }
    for (int c0 = 0; c0 < np_; c0 += kAccChunk) {
      const int n = min(kAccChunk, np_ - c0);
      load_records(first + c0, n);
      if (c0 > 0) __syncthreads();  // the previous chunk's carries and row flags are done
      for (int i = tid; i <= kBkPos; i += kAccThreads) cnt[i] = 0;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kAccPerThread; ++j)
        if (tid + j * kAccThreads < n) atomicAdd(&cnt[rq[j] & (kBkPos - 1)], 1);
      __syncthreads();
      {  // exclusive scan of the kBkPos counts, one per thread of waves 0-3
        int v = 0, incl = 0;
        if (tid < kBkPos) {
          v = cnt[tid];
          incl = v;
#pragma unroll
          for (int d = 1; d < kWave; d <<= 1) {
            const int t = __shfl_up(incl, d, kWave);
            if (lane >= d) incl += t;
          }
          if (lane == kWave - 1) wsum[wave] = incl;
        }
        __syncthreads();
        if (tid < kBkPos) {
          for (int w2 = 0; w2 < wave; ++w2) incl += wsum[w2];
          cur[tid] = incl - v;
        }
      }
      __syncthreads();
      if (tid < kBkPos) cnt[tid] = cur[tid];
      if (tid == 0) cnt[kBkPos] = n;
      __syncthreads();
#pragma unroll
      for (int j = 0; j < kAccPerThread; ++j)
        if (tid + j * kAccThreads < n) {
          const int slot = atomicAdd(&cur[rq[j] & (kBkPos - 1)], 1);
          lw[slot] = rw[j];
          lq[slot] = rq[j];
        }
      // group cut points: pcut[g] = the smallest position pp with cnt[pp] >= t_g = n * g / NGR
      // (whole positions per group; a chunk holds ~8 records per position)
      if constexpr (VEC == 4) {
        // fp32: position pp takes the groups with cnt[pp - 1] < t_g <= cnt[pp] (cnt[-1]
        // read as -1; t_g <= c exactly when g <= ((c + 1) * NGR - 1) / n), no dependent
        // LDS reads
        if (tid <= kBkPos) {
          const int hi = cnt[tid], lo = tid > 0 ? cnt[tid - 1] : -1;
          const int g0 = fast_div((lo + 1) * NGR + n - 1, n);  // operands < 2^24
          const int g1 = min(fast_div((hi + 1) * NGR - 1, n), NGR - 1);
          for (int g = g0; g <= g1; ++g) pcut[g] = tid;
        }
        if (tid == 0) pcut[NGR] = kBkPos;
      } else {
        // 16-bit types: a binary search per group (the form above measured slower here:
        // its registers push the 16-bit kernel's allocation into more spills)
        if (tid <= NGR) {
          const int target = n * tid / NGR;
          int lo = 0, hi = kBkPos;  // cnt[kBkPos] = n
          while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (cnt[mid] >= target) hi = mid; else lo = mid + 1;
          }
          pcut[tid] = tid == NGR ? kBkPos : lo;
        }
      }
      __syncthreads();
      const int p0 = pcut[gi], p1 = pcut[gi + 1];
      // sums of the group's current position and of the position after it
      float accl[VEC], accr[VEC];
#pragma unroll
      for (int c = 0; c < VEC; ++c) accl[c] = accr[c] = 0.f;
      bool carry = false;  // accr belongs to p1, the next group's first position
      // each row is written by one group during the walk: a plain store for a one-chunk
      // piece, an add to the earlier chunks' sums otherwise (rows that no record of the
      // piece reaches are never read)
      auto flush = [&](int at, float (&a)[VEC]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < VEC; c += 4) {
          float4 *dst = reinterpret_cast<float4 *>(&accs[at * D + cl * VEC + c]);
          float4 v = make_float4(a[c], a[c + 1], a[c + 2], a[c + 3]);
          if (multi) {
            const float4 o = *dst;
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
          }
          *dst = v;
        }
#pragma unroll
        for (int c = 0; c < VEC; ++c) a[c] = 0.f;
      };
      const int k0 = cnt[p0], k1 = cnt[p1];
      if (k0 < k1) {
        // records [k0, k1) of the group's positions, BT at a time (one 16-byte piece of
        // each record's grad_output row per lane), the next batch loaded while this one is
        // summed; a position without records gets no row from the walk (its row is written
        // by the carry of the group before it, or is never read)
        int pos = (int)(lq[k0] & (kBkPos - 1));
        float2 wa[BT], wb[BT];
        Vec<T, VEC> va[BT], vb[BT];
        int ra[BT], rb[BT];  // positions of the batch's records
        auto fetch = [&](int kk0, float2 (&w)[BT], Vec<T, VEC> (&v)[BT], int (&rp)[BT]) __attribute__((always_inline)) {
          uint32_t qv[BT];
#pragma unroll
          for (int u = 0; u < BT; ++u) {
            const int kk = min(kk0 + u, k1 - 1);
            w[u] = lw[kk];
            qv[u] = lq[kk];
          }
#pragma unroll
          for (int u = 0; u < BT; ++u) {
            rp[u] = (int)(qv[u] & (kBkPos - 1));
            v[u] = buffer_load_vec<T, VEC>(gr, (qv[u] >> kBkShift) * go_q_bytes + ch_bytes);
          }
        };
        auto consume = [&](int kk0, const float2 (&w)[BT], const Vec<T, VEC> (&v)[BT], const int (&rp)[BT]) __attribute__((always_inline)) {
#pragma unroll
          for (int u = 0; u < BT; ++u) {
            const int kk = kk0 + u;
            if (kk < k1) {
              if (rp[u] != pos) {  // record kk starts a later position of this group
                flush(pos, accl);
                const int np = rp[u];
                if (np == pos + 1) {
#pragma unroll
                  for (int c = 0; c < VEC; ++c) {
                    accl[c] = accr[c];
                    accr[c] = 0.f;
                  }
                } else {
                  flush(pos + 1, accr);  // no records there: this group's row
                }
                pos = np;
              }
#pragma unroll
              for (int c = 0; c < VEC; ++c) {
                const float g = (float)v[u].v[c];
                accl[c] += w[u].x * g;
                accr[c] += w[u].y * g;
              }
            }
          }
        };
        fetch(k0, wa, va, ra);
        int kk0 = k0;
        for (; kk0 + BT < k1; kk0 += 2 * BT) {
          fetch(kk0 + BT, wb, vb, rb);
          consume(kk0, wa, va, ra);
          if (kk0 + 2 * BT < k1) fetch(kk0 + 2 * BT, wa, va, ra);
          consume(kk0 + BT, wb, vb, rb);
        }
        if (kk0 < k1) consume(kk0, wa, va, ra);
        flush(pos, accl);
        if (pos + 1 < p1) flush(pos + 1, accr);
        else carry = true;
      }
      __syncthreads();  // every row of the walk is written
      if (carry) {  // p1: stored by its group this chunk if it has records, else not yet
        const bool keep = multi || has(p1);
#pragma unroll
        for (int c = 0; c < VEC; c += 4) {
          float4 *dst = reinterpret_cast<float4 *>(&accs[p1 * D + cl * VEC + c]);
          float4 v = make_float4(accr[c], accr[c + 1], accr[c + 2], accr[c + 3]);
          if (keep) {
            const float4 o = *dst;
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
          }
          *dst = v;
        }
      }
      if (multi && tid <= kBkPos && (has(tid) || (tid > 0 && has(tid - 1)))) touched[tid] = 1;
    }
    // the piece's rows, the next bucket's first included (positions past S do not exist;
    // rows no record reached are skipped): 4 channels per thread for the plain
    // read-modify-write; atomics on consecutive floats across the lanes (the L2 works per
    // line of each atomic instruction)
    float *gvb = p.gv + ((int64_t)b * p.S + (int64_t)kb * kBkPos) * (p.NH * D) + h * D;
    const int npos = min(kBkPos + 1, p.S - kb * kBkPos);
    __syncthreads();
    auto used = [&](int pp) __attribute__((always_inline)) {
      return multi ? touched[pp] != 0 : (has(pp) || (pp > 0 && has(pp - 1)));
    };
    if (whole) {
      for (int i = tid; i < npos * (D / 4); i += kAccThreads) {
        const int pp = i / (D / 4), c = (i - pp * (D / 4)) * 4;
        if (used(pp)) {
          const float4 v = *reinterpret_cast<const float4 *>(&accs[pp * D + c]);
          float *dst = gvb + (int64_t)pp * (p.NH * D) + c;
          if (pp == 0 || pp == kBkPos) {
            unsafeAtomicAdd(dst, v.x);
            unsafeAtomicAdd(dst + 1, v.y);
            unsafeAtomicAdd(dst + 2, v.z);
            unsafeAtomicAdd(dst + 3, v.w);
          } else {
            float4 o = *reinterpret_cast<const float4 *>(dst);
            o.x += v.x; o.y += v.y; o.z += v.z; o.w += v.w;
            *reinterpret_cast<float4 *>(dst) = o;
          }
        }
      }
    } else {
      for (int i = tid; i < npos * D; i += kAccThreads) {
        const int pp = i / D, c = i - pp * D;
        if (used(pp)) unsafeAtomicAdd(gvb + (int64_t)pp * (p.NH * D) + c, accs[i]);
      }
    }
    m = __builtin_amdgcn_readfirstlane(s_next);
  }
}

// grad_sampling_loc / grad_attn_weight for D = 32 without grad_value. A wave takes a tile
// of queries of one (batch, head) slice, `upi` units at a time (upi * L * P <= 64 samples,
// one per lane; more samples than 64 go in chunks of 64 with upi = 1):
//   1. lane i takes sample i: loads its location and attention weight, and writes the four
//      corner offsets (an out-of-range offset for a corner outside the level or a sample
//      outside the window, so the load returns zeros) and (lh, lw, a * H, a * W) to LDS;
//   2. groups of LPS lanes (LPS * 16 bytes = one corner row) take the samples in steps,
//      each group staying on one unit so that its grad_output piece stays in registers,
//      form S_k = sum_c top_c * v_k,c for the four corners, reduce the three gradients
//      (linear in S_k) over the group and leave them in LDS;
//   3. lane i stores sample i's gradients (contiguous stores).
// Tiles are ordered slice by slice and XCD x takes the x-th eighth of them, so the
// workgroups of one XCD gather from one slice of value at a time (a slice of the SCA map
// is 3.9 MB in fp32, the size of an XCD's L2).
constexpr int kCoWaves = 4;  // waves per workgroup
constexpr int kCoIters = 4;  // unit groups per tile

struct CoordParams {
  const void *value, *loc, *attn, *grad_out;
  void *grad_loc, *grad_attn;
  const int64_t *shapes, *lsi;
  int64_t go_sb, go_sq, go_sh;  // grad_output strides, elements (channels contiguous)
  int NH, NQ, NL, NP, S;
  int upi;     // units per pass
  int tps;     // tiles per slice
  int nt8;     // tiles per XCD
  int ntiles;
  const float *nsrc;  // 16-bit types: the fp32 grad_value workspace, narrowed into ndst
  void *ndst;         //   by the waves after their tiles (float4 groups; 0: none)
  int64_t nn4;
};

// Sum over each LPS-lane group (4 or 8) with DPP moves, no LDS traffic: xor 1 and xor 2
// inside each quad (quad_perm [1,0,3,2] and [2,3,0,1]); for 8 lanes, row_shr:4 then adds
// the lower quad's sum to the upper quad (lanes whose source is outside the 16-lane row
// read 0). Lane LPS - 1 of the group ends with the group's total.
template <int LPS>
__device__ __forceinline__ float group_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  if constexpr (LPS == 8)
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x114, 0xF, 0xF, true));
  return v;
}

// sum_c a_c * b_c over one 16-byte piece of a row, in fp32: fused multiply-adds for fp32,
// v_dot2 (two exact 16-bit products and an fp32 accumulator per instruction) for f16 / bf16
template <typename T, int VEC>
__device__ __forceinline__ float piece_dot(const Vec<T, VEC> &a, const Vec<T, VEC> &b) {
  if constexpr (sizeof(T) == 4) {
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < VEC; ++c) s = fmaf((float)a.v[c], (float)b.v[c], s);
    return s;
  } else if constexpr (std::is_same<T, f16>::value) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    struct P { h2 v[VEC / 2]; };
    const P pa = __builtin_bit_cast(P, a), pb = __builtin_bit_cast(P, b);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < VEC / 2; ++c) s = __builtin_amdgcn_fdot2(pa.v[c], pb.v[c], s, false);
    return s;
  } else {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    struct P { b2 v[VEC / 2]; };
    const P pa = __builtin_bit_cast(P, a), pb = __builtin_bit_cast(P, b);
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < VEC / 2; ++c) s = __builtin_amdgcn_fdot2_f32_bf16(pa.v[c], pb.v[c], s, false);
    return s;
  }
}

// LDS stores by one lane become visible to loads by other lanes of the same wave once
// issued (a wave's LDS instructions execute in order); this keeps the compiler from
// moving memory accesses across the hand-over.
__device__ __forceinline__ void wave_lds_handover() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
__global__ void __launch_bounds__(kCoWaves * kWave) msda_coord_kernel(const CoordParams p) {
  constexpr int D = 32, VEC = 16 / (int)sizeof(T), LPS = D / VEC, G = kWave / LPS;
  constexpr uint32_t kPast = 0x80000000u;
  __shared__ uint4 s_off[kCoWaves][kWave];   // corner byte offsets
  __shared__ float4 s_par[kCoWaves][kWave];  // lh, lw, a * H, a * W
  __shared__ float4 s_res[kCoWaves][kWave];  // grad_w, grad_h, grad_attn
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & (kWave - 1);
  const int xcd = blockIdx.x & 7, r = blockIdx.x >> 3;
  // the wave's tile is uniform: kept in scalar registers
  const int tloc = __builtin_amdgcn_readfirstlane(r * kCoWaves + wave);
  const int tile = xcd * p.nt8 + tloc;
  // 16-bit types: this wave's contiguous share of the fp32 grad_value workspace, narrowed
  // into grad_value after the wave's tile (the accumulate kernel ran before this kernel)
  auto narrow_share = [&]() __attribute__((always_inline)) {
    const int64_t nw = (int64_t)gridDim.x * kCoWaves;
    const int64_t per = (p.nn4 + nw - 1) / nw;
    const int64_t i0 = ((int64_t)blockIdx.x * kCoWaves + wave) * per;
    const int64_t i1 = min(i0 + per, p.nn4);
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int U = 4;  // loads in flight per lane: one memory latency per round
    for (int64_t i = i0 + lane; i < i1; i += U * kWave) {
      f4v v[U];
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i + u * kWave < i1)
          v[u] = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(p.nsrc) + i + u * kWave);
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (i + u * kWave < i1) {
          Vec<T, 4> o;
          o.v[0] = (T)v[u].x; o.v[1] = (T)v[u].y; o.v[2] = (T)v[u].z; o.v[3] = (T)v[u].w;
          store_vec_nt<T, 4>(static_cast<T *>(p.ndst) + 4 * (i + u * kWave), o);
        }
    }
  };
  if (tloc >= p.nt8 || tile >= p.ntiles) {
    if constexpr (sizeof(T) == 2) narrow_share();
    return;
  }
  const int slice = tile / p.tps;
  const int tq = tile - slice * p.tps;
  const int b = slice / p.NH, h = slice - b * p.NH;
  const int NS = p.NL * p.NP, upi = p.upi;
  const int q_begin = tq * upi * kCoIters, q_end = min(p.NQ, q_begin + upi * kCoIters);
  const int row = p.NH * D;
  const T *vb = static_cast<const T *>(p.value) + (int64_t)b * p.S * row + h * D;
  const __amdgpu_buffer_rsrc_t rv =
      make_rsrc(vb, (uint32_t)(((int64_t)p.S * row - h * D) * sizeof(T)));
  const T *loc = static_cast<const T *>(p.loc);
  const T *attn = static_cast<const T *>(p.attn);
  T *gloc = static_cast<T *>(p.grad_loc);
  T *gattn = static_cast<T *>(p.grad_attn);
  const T *gob = static_cast<const T *>(p.grad_out) + b * p.go_sb + h * p.go_sh;
  // group lanes: unit slot ug, sample column gq of GPU per unit, channels cl * VEC ..
  const int g = lane / LPS, cl = lane - g * LPS;
  const int ug = g % upi, gq = g / upi, GPU = G / upi;
  const uint32_t lane_b = (uint32_t)(cl * VEC * sizeof(T));
  for (int c0 = 0; c0 < NS; c0 += kWave) {
    const int nsc = upi > 1 ? NS : min(kWave, NS - c0);  // samples per unit in this pass
    // slot i = ui * stride + k holds sample k of unit slot ui; stride = the samples the
    // GPU groups of a unit take in `steps` steps (a multiple of GPU, upi * stride <= 64:
    // upi * nsc <= 64 and G divides 64); slots k >= nsc hold no sample (zero loads)
    const int steps = (nsc + GPU - 1) / GPU, stride = steps * GPU;
    // sample lanes: unit slot ui, sample s; the level geometry is fixed for the pass
    const int ui = lane / stride, k = lane - ui * stride, s = c0 + k;
    const bool lane_on = ui < upi && k < nsc;
    const int l = lane_on ? s / p.NP : 0;
    const int Hl = (int)p.shapes[2 * l], Wl = (int)p.shapes[2 * l + 1];
    const int lbase = (int)p.lsi[l];
    const float Hf = (float)Hl, Wf = (float)Wl;
    const uint32_t dx = (uint32_t)(row * sizeof(T)), dy = (uint32_t)(Wl * row * sizeof(T));
    // sample index of lane (ui, s) in the pass at q0: si0 + (q0 - q_begin) * NH * NS (32-bit:
    // the launch checks units * NS * 2 < 2^31); lanes past the units read sample 0 of unit 0
    const int uq = lane_on ? ui : 0;
    const int si0 = ((b * p.NQ + q_begin + uq) * p.NH + h) * NS + (lane_on ? s : c0);
    const int dsi = p.NH * NS;
    const int qlast = q_end - 1 - q_begin - uq;  // pass offset of the tile's last query
    // the next pass's location, attention weight and grad_output piece are loaded while
    // this pass runs
    Vec<T, 2> xy_n;
    T a_n;
    Vec<T, VEC> tv_n;
    auto fetch = [&](int q0) __attribute__((always_inline)) {
      const int si = si0 + min(q0 - q_begin, qlast) * dsi;
      xy_n = *reinterpret_cast<const Vec<T, 2> *>(loc + (int64_t)si * 2);
      a_n = attn[si];
      // fp32: grad_output pieces are read once here; streaming loads, like the gradient
      // stores below, keep the value lines in L2 (locations and weights stay ordinary
      // loads: streaming them was faster at SCA but slower at TSA; the 16-bit forms keep
      // ordinary accesses: streaming measured slower for TSA bf16)
      const int qg = min(q0 + ug, q_end - 1);
      if constexpr (sizeof(T) == 4)
        tv_n = load_vec_nt<T, VEC>(gob + (int64_t)qg * p.go_sq + cl * VEC);
      else
        tv_n = *reinterpret_cast<const Vec<T, VEC> *>(gob + (int64_t)qg * p.go_sq + cl * VEC);
    };
    fetch(q_begin);
    for (int q0 = q_begin; q0 < q_end; q0 += upi) {
      // 1. sample lanes
      const int qs = q0 + ui;
      const bool on = lane_on && qs < q_end;
      const int si = si0 + (q0 - q_begin) * dsi;
      const Vec<T, 2> xy = xy_n;
      const float a = (float)a_n;
      const Vec<T, VEC> top = tv_n;
      if (q0 + upi < q_end) fetch(q0 + upi);
      uint4 off = make_uint4(kPast, kPast, kPast, kPast);
      float4 par = make_float4(0.f, 0.f, 0.f, 0.f);
      float him, wim;
      sample_coords<float>((float)xy.v[0], (float)xy.v[1], Hl, Wl, him, wim);
      const bool win = on && him > -1.f && wim > -1.f && him < Hf && wim < Wf;
      if (win) {
        const float fh = floorf(him), fw = floorf(wim);
        const int hl = (int)fh, wl = (int)fw;
        const uint32_t e1 = (uint32_t)((lbase + hl * Wl + wl) * row) * (uint32_t)sizeof(T);
        const bool y0 = hl >= 0, y1 = hl + 1 <= Hl - 1, x0 = wl >= 0, x1 = wl + 1 <= Wl - 1;
        off.x = y0 && x0 ? e1 : kPast;
        off.y = y0 && x1 ? e1 + dx : kPast;
        off.z = y1 && x0 ? e1 + dy : kPast;
        off.w = y1 && x1 ? e1 + dy + dx : kPast;
        par = make_float4(him - fh, wim - fw, a * Hf, a * Wf);
      }
      s_off[wave][lane] = off;
      s_par[wave][lane] = par;
      wave_lds_handover();
      // 2. group lanes, two steps at a time (a step past `steps` reads slot 0 of its unit
      // again and writes the same result there)
      for (int t = 0; t < steps; t += 2) {
        Vec<T, VEC> cv[2][4];
        float4 pr[2];
        int slot[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int tj = t + j < steps ? t + j : 0;
          slot[j] = ug * stride + tj * GPU + gq;
          const uint4 o = s_off[wave][slot[j]];
          pr[j] = s_par[wave][slot[j]];
          cv[j][0] = buffer_load_vec<T, VEC>(rv, o.x + lane_b);
          cv[j][1] = buffer_load_vec<T, VEC>(rv, o.y + lane_b);
          cv[j][2] = buffer_load_vec<T, VEC>(rv, o.z + lane_b);
          cv[j][3] = buffer_load_vec<T, VEC>(rv, o.w + lane_b);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const float s1 = piece_dot<T, VEC>(top, cv[j][0]), s2 = piece_dot<T, VEC>(top, cv[j][1]);
          const float s3 = piece_dot<T, VEC>(top, cv[j][2]), s4 = piece_dot<T, VEC>(top, cv[j][3]);
          const float lh = pr[j].x, lw = pr[j].y, hh = 1.f - lh, hw = 1.f - lw;
          // a sample outside the window has no valid corner (its sums are discarded below)
          float gh = pr[j].z * (hw * (s3 - s1) + lw * (s4 - s2));
          float gw = pr[j].w * (hh * (s2 - s1) + lh * (s4 - s3));
          float ga = hh * hw * s1 + hh * lw * s2 + lh * hw * s3 + lh * lw * s4;
          gh = group_sum<LPS>(gh);
          gw = group_sum<LPS>(gw);
          ga = group_sum<LPS>(ga);
          if (cl == LPS - 1) s_res[wave][slot[j]] = make_float4(gw, gh, ga, 0.f);
        }
      }
      wave_lds_handover();
      // 3. sample lanes; a sample outside its level writes zeros whatever grad_output holds
      // (the reference skips it: ms_deform_attn_kernels.cuh:252-259)
      if (on) {
        const float4 rr = win ? s_res[wave][lane] : make_float4(0.f, 0.f, 0.f, 0.f);
        Vec<T, 2> gl;
        gl.v[0] = (T)rr.x;
        gl.v[1] = (T)rr.y;
        if constexpr (sizeof(T) == 4) {
          store_vec_nt<T, 2>(gloc + (int64_t)si * 2, gl);
          __builtin_nontemporal_store((T)rr.z, gattn + si);
        } else {
          *reinterpret_cast<Vec<T, 2> *>(gloc + (int64_t)si * 2) = gl;
          gattn[si] = (T)rr.z;
        }
      }
      wave_lds_handover();
    }
  }
  if constexpr (sizeof(T) == 2) narrow_share();
}

// Streaming passes over the fp32 grad_value workspace: 16-byte accesses when the
// pointers allow them, element by element for the rest.
__global__ void __launch_bounds__(kBlock) fill_zero_f32(float *__restrict__ p, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int64_t i0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const int64_t nv = reinterpret_cast<uintptr_t>(p) % 16 == 0 ? n / 4 : 0;
  for (int64_t i = i0; i < nv; i += stride)
    reinterpret_cast<float4 *>(p)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int64_t i = nv * 4 + i0; i < n; i += stride) p[i] = 0.f;
}

template <typename T>
__global__ void __launch_bounds__(kBlock) narrow_f32(const float *__restrict__ src,
                                                     T *__restrict__ dst, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * kBlock;
  const int64_t i0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  const bool vec = reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(dst) % (4 * sizeof(T)) == 0;
  const int64_t nv = vec ? n / 4 : 0;
  for (int64_t i = i0; i < nv; i += stride) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    const f4v v = __builtin_nontemporal_load(reinterpret_cast<const f4v *>(src) + i);
    Vec<T, 4> o;
    o.v[0] = (T)v.x; o.v[1] = (T)v.y; o.v[2] = (T)v.z; o.v[3] = (T)v.w;
    store_vec_nt<T, 4>(dst + 4 * i, o);
  }
  for (int64_t i = nv * 4 + i0; i < n; i += stride) dst[i] = (T)src[i];
}

unsigned stream_grid(int64_t n) {
  const int64_t g = (n + kBlock - 1) / kBlock;
  return (unsigned)(g < 8192 ? (g > 0 ? g : 1) : 8192);
}

// Workspace of the sorted grad_value path (bytes, after the 16-bit accumulator).
struct BktLayout {
  int NBS = 0, nbk = 0, item_cap = 0;
  int64_t cap = 0;  // record slots (two per sample)
  int64_t off_count = 0, off_cursor = 0, off_offset = 0, off_nitems = 0, off_items = 0,
          off_rw = 0, off_rq = 0, bytes = 0;
};

BktLayout bkt_layout(int64_t B, int64_t S, int64_t NH, int64_t NL, int64_t NQ, int64_t NP) {
  BktLayout L;
  auto up = [](int64_t x) { return (x + 255) / 256 * 256; };
  const int64_t nbs = (S + kBkPos - 1) / kBkPos;
  const int64_t cap = B * NQ * NH * NL * NP * 2;
  const int64_t nbk = B * NH * nbs;
  const int64_t item_cap = (cap + kAccChunk - 1) / kAccChunk + nbk;  // chunks of one list
  if (nbs <= 0 || nbs > kBkMaxPerSlice || cap <= 0 || cap >= ((int64_t)1 << 31) ||
      nbk >= ((int64_t)1 << 26) || item_cap >= ((int64_t)1 << 26) || NQ >= ((int64_t)1 << 22) ||
      NL * NP > kChunkSamples)
    return L;  // bytes == 0: not applicable
  L.NBS = (int)nbs; L.nbk = (int)nbk; L.item_cap = (int)item_cap; L.cap = cap;
  int64_t o = 0;
  L.off_count = o;  o += up(nbk * 4);
  L.off_cursor = o; o += up(nbk * 4);
  L.off_offset = o; o += up((nbk + 1) * 4);
  L.off_nitems = o; o += up(8 * 4);
  L.off_items = o;  o += up(8 * item_cap * 16);
  L.off_rw = o;     o += up(cap * 8);
  L.off_rq = o;     o += up(cap * 4);
  L.bytes = o;
  return L;
}

int64_t half_acc_bytes(int dtype, int64_t value_elems) {
  return (dtype == 1 || dtype == 2) ? (value_elems * (int64_t)sizeof(float) + 255) / 256 * 256 : 0;
}

// The sorted path: D = 32, fp32 accumulation (f32 / f16 / bf16 inputs), one batch of value
// under 2 GiB (32-bit buffer offsets), and a workspace that holds its buffers.
template <typename T>
bool sorted_path(const MsdaBwdArgs &a, int dtype, BktLayout &L) {
  if (a.f.channels != 32 || a.f.batch <= 0 || a.f.num_heads <= 0 || a.f.num_query <= 0 ||
      a.f.num_levels <= 0 || a.f.num_point <= 0 || device_cus() < 8)
    return false;
  if ((int64_t)a.f.spatial_size * a.f.num_heads * 32 * (int64_t)sizeof(T) >= ((int64_t)1 << 31))
    return false;
  if ((int64_t)a.f.batch * a.f.num_query * a.f.num_heads >= ((int64_t)1 << 31) / 64) return false;
  // sample indices of loc / grad_loc in 32 bits
  if ((int64_t)a.f.batch * a.f.num_query * a.f.num_heads * a.f.num_levels * a.f.num_point * 2 >=
      ((int64_t)1 << 31))
    return false;
  // 16-byte corner rows; (x, y) pairs of loc / grad_loc read and written as one access
  if (reinterpret_cast<uintptr_t>(a.f.value) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(a.f.sampling_loc) % (2 * sizeof(T)) != 0 ||
      reinterpret_cast<uintptr_t>(a.grad_loc) % (2 * sizeof(T)) != 0 ||
      reinterpret_cast<uintptr_t>(a.grad_value) % 16 != 0)
    return false;
  // grad_output rows through 32-bit buffer offsets
  // (16-byte pieces of grad_output rows: contiguous channels, aligned rows)
  if (reinterpret_cast<uintptr_t>(a.grad_output) % 16 != 0 || a.go_stride[0] < 0 ||
      a.go_stride[2] < 0 || (a.go_stride[0] * (int64_t)sizeof(T)) % 16 != 0 ||
      (a.go_stride[2] * (int64_t)sizeof(T)) % 16 != 0)
    return false;
  if (a.go_stride[1] < 0 || a.go_stride[3] != 1 || (a.go_stride[1] * (int64_t)sizeof(T)) % 16 != 0 ||
      ((int64_t)(a.f.num_query - 1) * a.go_stride[1] + 31 * a.go_stride[3] + 1) * (int64_t)sizeof(T) >=
          ((int64_t)1 << 31))
    return false;
  L = bkt_layout(a.f.batch, a.f.spatial_size, a.f.num_heads, a.f.num_levels, a.f.num_query,
                 a.f.num_point);
  if (L.bytes == 0) return false;
  const int64_t value_elems = (int64_t)a.f.batch * a.f.spatial_size * a.f.num_heads * 32;
  return a.workspace != nullptr &&
         a.workspace_bytes >= half_acc_bytes(dtype, value_elems) + L.bytes;
}

// grad_value (fp32, added to gv) by the four bucket kernels, then the coordinate kernel.
// fused_n: 16-bit types with a 16-byte aligned fp32 workspace gv and an 8-byte aligned
// grad_value: the workspace's element count; the count kernel clears gv and the coordinate
// kernel narrows it into grad_value. 0: gv is the caller's fp32 grad_value, or the
// caller clears and narrows.
template <typename T>
hipError_t launch_sorted(const MsdaBwdArgs &a, const BktLayout &L, char *ws, float *gv,
                         int64_t fused_n, hipStream_t stream) {
  BktParams p;
  p.loc = a.f.sampling_loc;
  p.attn = a.f.attn_weight;
  p.grad_out = a.grad_output;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.gv = gv;
  p.count = reinterpret_cast<int *>(ws + L.off_count);
  p.cursor = reinterpret_cast<int *>(ws + L.off_cursor);
  p.offset = reinterpret_cast<int *>(ws + L.off_offset);
  p.nitems = reinterpret_cast<int *>(ws + L.off_nitems);
  p.items = reinterpret_cast<int4 *>(ws + L.off_items);
  p.rw = reinterpret_cast<float2 *>(ws + L.off_rw);
  p.rq = reinterpret_cast<uint32_t *>(ws + L.off_rq);
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.B = a.f.batch; p.NH = a.f.num_heads; p.NQ = a.f.num_query; p.NL = a.f.num_levels;
  p.NP = a.f.num_point; p.S = a.f.spatial_size;
  p.go_rows_bytes = (uint32_t)(((int64_t)(a.f.num_query - 1) * a.go_stride[1] + 31 * a.go_stride[3] + 1) *
                               (int64_t)sizeof(T));
  p.NBS = L.NBS; p.nbk = L.nbk; p.item_cap = L.item_cap;
  p.by_bucket = (int64_t)a.f.batch * a.f.num_heads < 8 ? 1 : 0;
  const int blocks = (device_cus() / 8) * 8 * 2;  // two 8-wave workgroups per CU (LDS)
  p.blocks_per_xcd = blocks / 8;
  p.qpb = kChunkSamples / (a.f.num_levels * a.f.num_point);
  const int qchunks = (a.f.num_query + p.qpb - 1) / p.qpb;
  p.cblk8 = (int)(((int64_t)a.f.batch * a.f.num_heads * qchunks + 7) / 8);
  // persistent count blocks: 8 per CU (4 KB LDS each); place blocks: 4 per CU (36 KB)
  const int cus8 = device_cus() / 8;
  const int count_pblk = std::max(1, std::min(p.cblk8, cus8 * 8));
  const int place_pblk = std::max(1, std::min(p.cblk8, cus8 * 4));
  hipLaunchKernelGGL(fill_zero_f32, dim3(stream_grid(L.nbk)), dim3(kBlock), 0, stream,
                     reinterpret_cast<float *>(p.count), (int64_t)L.nbk);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  p.pblk = count_pblk;
  p.zero = fused_n > 0 ? gv : nullptr;
  p.nzero4 = fused_n / 4;
  hipLaunchKernelGGL((msda_bkt_count_kernel<T>), dim3(8u * (unsigned)count_pblk), dim3(kBkThreads), 0,
                     stream, p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(msda_bkt_scan_kernel, dim3(8), dim3(1024), 0, stream, p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  p.pblk = place_pblk;
  hipLaunchKernelGGL((msda_bkt_place_kernel<T>), dim3(8u * (unsigned)place_pblk), dim3(kBkThreads), 0,
                     stream, p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL((msda_bkt_acc_kernel<T>), dim3(blocks), dim3(kAccThreads), 0, stream, p);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  CoordParams c;
  c.value = a.f.value;
  c.loc = a.f.sampling_loc;
  c.attn = a.f.attn_weight;
  c.grad_out = a.grad_output;
  c.grad_loc = a.grad_loc;
  c.grad_attn = a.grad_attn;
  c.shapes = a.f.spatial_shapes;
  c.lsi = a.f.level_start_index;
  c.go_sb = a.go_stride[0]; c.go_sq = a.go_stride[1]; c.go_sh = a.go_stride[2];
  c.NH = a.f.num_heads; c.NQ = a.f.num_query; c.NL = a.f.num_levels; c.NP = a.f.num_point;
  c.S = a.f.spatial_size;
  const int ns = a.f.num_levels * a.f.num_point;
  c.upi = ns <= 16 ? 4 : ns <= 32 ? 2 : 1;
  c.tps = (a.f.num_query + c.upi * kCoIters - 1) / (c.upi * kCoIters);
  const int64_t ntiles = (int64_t)a.f.batch * a.f.num_heads * c.tps;
  c.ntiles = (int)ntiles;
  c.nt8 = (int)((ntiles + 7) / 8);
  c.nsrc = gv;
  c.ndst = a.grad_value;
  c.nn4 = fused_n / 4;
  const unsigned cgrid = 8u * (unsigned)((c.nt8 + kCoWaves - 1) / kCoWaves);
  hipLaunchKernelGGL((msda_coord_kernel<T>), dim3(cgrid), dim3(kCoWaves * kWave), 0, stream, c);
  return hipGetLastError();
}

// One-level grid with one query per cell, D = 32, at most kOwnMaxP points: grad_value by
// the owner pass (every element written) plus far samples' atomics.
// (16-byte aligned value, one batch of value under 2 GiB for the 31-bit buffer offsets.)
template <typename T>
bool owner_path(const MsdaBwdArgs &a) {
  return a.f.num_levels == 1 && a.f.num_query == a.f.spatial_size && a.f.channels == 32 &&
         a.f.num_point >= 1 && a.f.num_point <= kOwnMaxP && a.f.spatial_size > 0 &&
         reinterpret_cast<uintptr_t>(a.f.value) % 16 == 0 &&
         (int64_t)a.f.spatial_size * a.f.num_heads * 32 * (int64_t)sizeof(T) < ((int64_t)1 << 31) &&
         (int64_t)a.f.batch * a.f.num_query * a.f.num_heads * 8 < ((int64_t)1 << 31) &&
         (int64_t)a.f.batch * a.f.num_query < ((int64_t)1 << 22) && device_cus() >= 8;
}

template <typename T>
hipError_t launch_owner(const MsdaBwdArgs &a, float *gv, bool accumulate, hipStream_t stream) {
  OwnParams p;
  p.accumulate = accumulate ? 1 : 0;
  p.loc = a.f.sampling_loc;
  p.attn = a.f.attn_weight;
  p.grad_out = a.grad_output;
  p.gv = gv;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.B = a.f.batch; p.NH = a.f.num_heads; p.NQ = a.f.num_query; p.NP = a.f.num_point;
  p.S = a.f.spatial_size;
  const int blocks = (device_cus() / 8) * 8 * 2;  // two 8-wave workgroups per CU
  p.blocks_per_xcd = blocks / 8;
  if (a.f.batch == 0 || a.f.num_heads == 0) return hipSuccess;
  switch (a.f.num_point) {
    case 1: hipLaunchKernelGGL((msda_gv_owner_kernel<T, 1>), dim3(blocks), dim3(kOwnThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((msda_gv_owner_kernel<T, 2>), dim3(blocks), dim3(kOwnThreads), 0, stream, p); break;
    case 3: hipLaunchKernelGGL((msda_gv_owner_kernel<T, 3>), dim3(blocks), dim3(kOwnThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL((msda_gv_owner_kernel<T, 4>), dim3(blocks), dim3(kOwnThreads), 0, stream, p); break;
  }
  return hipGetLastError();
}

// The coarse split (msda_coarse_gv_kernel + msda_col2im_kernel without the coarse levels'
// atomics) for D = 32 and fp32 accumulation.
template <typename T, typename A>
bool coarse_split(const MsdaBwdArgs &a) {
  return sizeof(A) == 4 && a.f.channels == 32 && a.f.num_levels >= 1 && device_cus() >= 8 &&
         a.f.num_query > 0 && a.f.batch > 0 && a.f.num_heads > 0 &&
         a.f.num_levels * a.f.num_point <= kCoarseMaxSPU;
}

template <typename T>
hipError_t launch_coarse(const MsdaBwdArgs &a, float *gv, hipStream_t stream) {
  CoarseParams p;
  p.loc = a.f.sampling_loc;
  p.attn = a.f.attn_weight;
  p.grad_out = a.grad_output;
  p.gv = gv;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.B = a.f.batch; p.NH = a.f.num_heads; p.NQ = a.f.num_query; p.NL = a.f.num_levels;
  p.NP = a.f.num_point; p.S = a.f.spatial_size;
  const int blocks = (device_cus() / 8) * 8;  // one 8-wave workgroup per CU (LDS)
  p.blocks_per_xcd = blocks / 8;
  hipLaunchKernelGGL((msda_coarse_gv_kernel<T>), dim3(blocks), dim3(kCoarseThreads), 0, stream, p);
  return hipGetLastError();
}

// generic: the per-unit kernel alone (msda_col2im_kernel, every level's grad_value by
// atomics), the reference's force_generic_col2im.
template <typename T, typename A>
hipError_t launch_t(const MsdaBwdArgs &a, A *grad_value, bool generic, hipStream_t stream) {
  BwdParams p;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.units = (int64_t)a.f.batch * a.f.num_query * a.f.num_heads;
  p.S = a.f.spatial_size; p.NH = a.f.num_heads; p.D = a.f.channels;
  p.NL = a.f.num_levels; p.NQ = a.f.num_query; p.NP = a.f.num_point;
  p.coarse = !generic && coarse_split<T, A>(a) ? 1 : 0;
  p.log2_g = 0;
  while ((1 << p.log2_g) < a.f.channels && p.log2_g < 6) ++p.log2_g;
  const int64_t threads = p.units << p.log2_g;
  if (threads == 0) return hipSuccess;
  if constexpr (sizeof(A) == 4) {
    if (p.coarse) {
      const hipError_t e = launch_coarse<T>(a, grad_value, stream);
      if (e != hipSuccess) return e;
    }
    if (!generic && a.f.channels == 32 && p.units * 32 < ((int64_t)1 << 31) &&
        (int64_t)a.f.batch * a.f.num_query < ((int64_t)1 << 22) &&
        (int64_t)a.f.spatial_size * a.f.num_heads * 32 * (int64_t)sizeof(T) < ((int64_t)1 << 31)) {
      hipLaunchKernelGGL((msda_col2im_d32_kernel<T>),
                         dim3((unsigned)((p.units * 32 + kBlock - 1) / kBlock)), dim3(kBlock), 0,
                         stream, static_cast<const T *>(a.f.value),
                         static_cast<const T *>(a.f.sampling_loc),
                         static_cast<const T *>(a.f.attn_weight),
                         static_cast<const T *>(a.grad_output), grad_value,
                         static_cast<T *>(a.grad_loc), static_cast<T *>(a.grad_attn), p);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL((msda_col2im_kernel<T, A>),
                     dim3((unsigned)((threads + kBlock - 1) / kBlock)), dim3(kBlock), 0, stream,
                     static_cast<const T *>(a.f.value), static_cast<const T *>(a.f.sampling_loc),
                     static_cast<const T *>(a.f.attn_weight),
                     static_cast<const T *>(a.grad_output), grad_value,
                     static_cast<T *>(a.grad_loc), static_cast<T *>(a.grad_attn), p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_grid_coord(const MsdaBwdArgs &a, float *gv, hipStream_t stream) {
  BwdParams p;
  p.shapes = a.f.spatial_shapes;
  p.lsi = a.f.level_start_index;
  p.go_sb = a.go_stride[0]; p.go_sq = a.go_stride[1];
  p.go_sh = a.go_stride[2]; p.go_sc = a.go_stride[3];
  p.units = (int64_t)a.f.batch * a.f.num_query * a.f.num_heads;
  p.S = a.f.spatial_size; p.NH = a.f.num_heads; p.D = a.f.channels;
  p.NL = a.f.num_levels; p.NQ = a.f.num_query; p.NP = a.f.num_point;
  p.coarse = 0;
  p.log2_g = 0;
  constexpr int G = 32 * (int)sizeof(T) / 16;
  const int64_t threads = p.units * G;
  if (threads == 0) return hipSuccess;
  hipLaunchKernelGGL((msda_grid_coord_kernel<T>), dim3((unsigned)((threads + kBlock - 1) / kBlock)),
                     dim3(kBlock), 0, stream, static_cast<const T *>(a.f.value),
                     static_cast<const T *>(a.f.sampling_loc), static_cast<const T *>(a.f.attn_weight),
                     static_cast<const T *>(a.grad_output), gv, static_cast<T *>(a.grad_loc),
                     static_cast<T *>(a.grad_attn), p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_f32(const MsdaBwdArgs &a, bool generic, hipStream_t stream) {
  float *gv = static_cast<float *>(a.grad_value);
  BktLayout L;
  if (!generic && sorted_path<T>(a, 0, L))
    return launch_sorted<T>(a, L, static_cast<char *>(a.workspace), gv, 0, stream);
  if (generic || !owner_path<T>(a)) return launch_t<T, float>(a, gv, generic, stream);
  hipError_t e = launch_owner<T>(a, gv, true, stream);
  if (e != hipSuccess) return e;
  return launch_grid_coord<T>(a, gv, stream);
}

template <typename T>
hipError_t launch_half(const MsdaBwdArgs &a, bool generic, hipStream_t stream) {
  const int64_t n = (int64_t)a.f.batch * a.f.spatial_size * a.f.num_heads * a.f.channels;
  float *acc = static_cast<float *>(a.workspace);
  hipError_t e;
  BktLayout L;
  const int dtype = std::is_same<T, f16>::value ? 1 : 2;
  if (!generic && sorted_path<T>(a, dtype, L)) {
    // the clear and the narrowing run inside the count and coordinate kernels when the
    // pointers allow 16- and 8-byte accesses (n is a multiple of 32 here)
    const bool fuse = reinterpret_cast<uintptr_t>(acc) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(a.grad_value) % (4 * sizeof(T)) == 0;
    if (!fuse) {
      hipLaunchKernelGGL(fill_zero_f32, dim3(stream_grid(n)), dim3(kBlock), 0, stream, acc, n);
      e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    e = launch_sorted<T>(a, L, static_cast<char *>(a.workspace) + half_acc_bytes(dtype, n), acc,
                         fuse ? n : 0, stream);
    if (e != hipSuccess || fuse) return e;
  } else if (!generic && owner_path<T>(a)) {  // the owner pass writes every element of the workspace
    e = launch_owner<T>(a, acc, false, stream);
    if (e != hipSuccess) return e;
    e = launch_grid_coord<T>(a, acc, stream);
  } else {
    hipLaunchKernelGGL(fill_zero_f32, dim3(stream_grid(n)), dim3(kBlock), 0, stream, acc, n);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_t<T, float>(a, acc, generic, stream);
  }
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((narrow_f32<T>), dim3(stream_grid(n)), dim3(kBlock), 0, stream, acc,
                     static_cast<T *>(a.grad_value), n);
  return hipGetLastError();
}

}  // namespace

int64_t msda_backward_workspace_min(int dtype, int64_t value_elems) {
  return (dtype == 1 || dtype == 2) ? value_elems * (int64_t)sizeof(float) : 0;
}

int64_t msda_backward_workspace_bytes(int dtype, int64_t batch, int64_t spatial_size,
                                      int64_t num_heads, int64_t channels, int64_t num_levels,
                                      int64_t num_query, int64_t num_point) {
  const int64_t value_elems = batch * spatial_size * num_heads * channels;
  if (dtype == 3 || channels != 32) return msda_backward_workspace_min(dtype, value_elems);
  const BktLayout L = bkt_layout(batch, spatial_size, num_heads, num_levels, num_query, num_point);
  if (L.bytes == 0) return msda_backward_workspace_min(dtype, value_elems);
  return half_acc_bytes(dtype, value_elems) + L.bytes;
}

hipError_t launch_msda_backward(int dtype, const MsdaBwdArgs &a, bool force_generic,
                                hipStream_t stream) {
  switch (dtype) {
    case 0: return launch_f32<float>(a, force_generic, stream);
    case 1: return launch_half<f16>(a, force_generic, stream);
    case 2: return launch_half<bf16>(a, force_generic, stream);
    case 3:
      return launch_t<double, double>(a, static_cast<double *>(a.grad_value), true, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace bevk
