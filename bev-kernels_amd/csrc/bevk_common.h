// Device-side helpers shared by the libbevk kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace bevk {

using f16 = _Float16;
using bf16 = __bf16;

constexpr int kWave = 64;

// Accumulation type: fp32 for every floating type except fp64.
template <typename T> struct Acc { using type = float; };
template <> struct Acc<double> { using type = double; };

template <typename A, typename T> __device__ __forceinline__ A cvt(T x) { return static_cast<A>(x); }

// Round-to-nearest-even conversions; gfx950 has native cvt instructions for both.
template <typename T> __device__ __forceinline__ T from_acc(float x) { return static_cast<T>(x); }
template <> __device__ __forceinline__ double from_acc<double>(float x) { return x; }

// Plain vector of N elements of T, loaded/stored as one memory instruction.
template <typename T, int N> struct alignas(sizeof(T) * N) Vec { T v[N]; };

template <typename T, int N>
__device__ __forceinline__ Vec<T, N> load_vec(const T *p) {
  return *reinterpret_cast<const Vec<T, N> *>(p);
}
template <typename T, int N>
__device__ __forceinline__ void store_vec(T *p, const Vec<T, N> &v) {
  *reinterpret_cast<Vec<T, N> *>(p) = v;
}
// Streaming store: the output is written once and never re-read by the kernel, so
// it should not evict the gather working set from L2.
template <typename T, int N>
__device__ __forceinline__ void store_vec_nt(T *p, const Vec<T, N> &v) {
  if constexpr (sizeof(Vec<T, N>) == 16) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    __builtin_nontemporal_store(*reinterpret_cast<const i4 *>(&v), reinterpret_cast<i4 *>(p));
  } else if constexpr (sizeof(Vec<T, N>) == 8) {
    typedef int i2 __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(*reinterpret_cast<const i2 *>(&v), reinterpret_cast<i2 *>(p));
  } else if constexpr (sizeof(Vec<T, N>) == 4) {
    __builtin_nontemporal_store(*reinterpret_cast<const int *>(&v), reinterpret_cast<int *>(p));
  } else {
    store_vec<T, N>(p, v);
  }
}

template <typename T> __device__ __forceinline__ T load_nt(const T *p) {
  return __builtin_nontemporal_load(p);
}
// Streaming load of a 4-, 8- or 16-byte vector (read once by the kernel).
template <typename T, int N>
__device__ __forceinline__ Vec<T, N> load_vec_nt(const T *p) {
  if constexpr (sizeof(Vec<T, N>) == 16) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const i4 *>(p)));
  } else if constexpr (sizeof(Vec<T, N>) == 8) {
    typedef int i2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const i2 *>(p)));
  } else {
    static_assert(sizeof(Vec<T, N>) == 4, "4-, 8- or 16-byte vectors");
    return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const int *>(p)));
  }
}
template <> __device__ __forceinline__ f16 load_nt<f16>(const f16 *p) {
  unsigned short u = __builtin_nontemporal_load(reinterpret_cast<const unsigned short *>(p));
  return __builtin_bit_cast(f16, u);
}
template <> __device__ __forceinline__ bf16 load_nt<bf16>(const bf16 *p) {
  unsigned short u = __builtin_nontemporal_load(reinterpret_cast<const unsigned short *>(p));
  return __builtin_bit_cast(bf16, u);
}

// Raw buffer resource over [base, base + bytes). Loads at offsets >= bytes return 0
// and make no memory request; the kernels use that for zero-padded gathers.
constexpr int kBufferDword3 = 0x00020000;  // raw buffer, 32-bit data format (gfx9 family)

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                           kBufferDword3);
}

// 16-byte (or 8/4-byte) raw buffer load returning VEC elements of T.
template <typename T, int VEC>
__device__ __forceinline__ Vec<T, VEC> buffer_load_vec(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  constexpr int bytes = sizeof(T) * VEC;
  Vec<T, VEC> out;
  if constexpr (bytes == 16) {
    typedef int i4 __attribute__((ext_vector_type(4)));
    i4 raw = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
    out = __builtin_bit_cast(Vec<T, VEC>, raw);
  } else if constexpr (bytes == 8) {
    typedef int i2 __attribute__((ext_vector_type(2)));
    i2 raw = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    out = __builtin_bit_cast(Vec<T, VEC>, raw);
  } else {
    static_assert(bytes == 4, "unsupported vector width");
    int raw = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
    out = __builtin_bit_cast(Vec<T, VEC>, raw);
  }
  return out;
}

// One element of T through the buffer path.
template <typename T>
__device__ __forceinline__ T buffer_load_one(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(T) == 8) {
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  } else if constexpr (sizeof(T) == 4) {
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  } else {
    static_assert(sizeof(T) == 2, "unsupported element size");
    return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  }
}

// Logistic function on the device exp; used where a raw offset-conv output carries
// the pre-sigmoid mask.
__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + __expf(-x)); }

// Sample geometry forms of the fused DCN kernels.
enum DcnGeo {
  kGeoMask = 0,     // offsets [M][2T] + mask [M][T], input dtype
  kGeoY = 1,        // raw offset-conv output y [M][3T], input dtype; mask = sigmoid(y[2T + t])
  kGeoRegular = 2,  // no offsets: a plain convolution (fp32 output; the offset conv)
  kGeoYF32 = 3,     // y [M][3T] fp32 (+ fp32 bias [3T] when given); mask = sigmoid
};

// Offsets (dy, dx) and mask of tap t of output row m in the deformable forms
// (dcn_fused_nhwc_kernel.cuh:126-134 and dcn_split_nhwc.py:131-132 for the y forms:
// offset = y[..., :2T] with (dy, dx) interleaved per tap, mask = sigmoid(y[..., 2T:])).
template <typename T, int GEO>
__device__ __forceinline__ void tap_offsets(const void *off, const void *msk, const float *yb,
                                            int64_t m, int t, int taps, float &dy, float &dx,
                                            float &mk) {
  if constexpr (GEO == kGeoY) {
    const T *yp = static_cast<const T *>(off) + m * 3 * taps;
    dy = (float)yp[2 * t];
    dx = (float)yp[2 * t + 1];
    mk = sigmoid_f32((float)yp[2 * taps + t]);
  } else if constexpr (GEO == kGeoYF32) {
    const float *yp = static_cast<const float *>(off) + m * 3 * taps;
    float b0 = 0.f, b1 = 0.f, b2 = 0.f;
    if (yb != nullptr) {
      b0 = yb[2 * t];
      b1 = yb[2 * t + 1];
      b2 = yb[2 * taps + t];
    }
    dy = yp[2 * t] + b0;
    dx = yp[2 * t + 1] + b1;
    mk = sigmoid_f32(yp[2 * taps + t] + b2);
  } else {
    const T *op = static_cast<const T *>(off);
    dy = (float)op[m * 2 * taps + 2 * t];
    dx = (float)op[m * 2 * taps + 2 * t + 1];
    mk = (float)static_cast<const T *>(msk)[m * taps + t];
  }
}

}  // namespace bevk
