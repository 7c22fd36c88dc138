// Shared helpers for the gfx950 MedNeXt kernels: element types, conversions,
// the per-thread error slot behind mednext_hip_last_error(), and launch checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>

#include "../../include/mednext_hip.h"

namespace mednext {

// Storage types. bf16 is kept as raw 16-bit words so conversions are explicit
// and identical on host and device.
struct bf16_t {
  uint16_t bits;
};
using f16_t = _Float16;

__host__ __device__ inline float bf16_to_f32(uint16_t b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN stays NaN, quiet bit forced).
__host__ __device__ inline uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0u) {
    return static_cast<uint16_t>((u >> 16) | 0x0040u);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// Load one element as the accumulation type, and store an accumulator back.
template <typename T, typename Acc>
struct Cvt;

template <>
struct Cvt<float, float> {
  __device__ static float load(float v) { return v; }
  __device__ static float store(float v) { return v; }
};
template <>
struct Cvt<double, double> {
  __device__ static double load(double v) { return v; }
  __device__ static double store(double v) { return v; }
};
template <>
struct Cvt<f16_t, float> {
  __device__ static float load(f16_t v) { return static_cast<float>(v); }
  __device__ static f16_t store(float v) { return static_cast<f16_t>(v); }
};
template <>
struct Cvt<bf16_t, float> {
  __device__ static float load(bf16_t v) { return bf16_to_f32(v.bits); }
  __device__ static bf16_t store(float v) { return bf16_t{f32_to_bf16(v)}; }
};

// Accumulation type per storage type: fp64 accumulates in fp64, the rest in fp32.
template <typename T>
struct AccOf {
  using type = float;
};
template <>
struct AccOf<double> {
  using type = double;
};

// a * b + c with one rounding in the accumulation type (written out so that
// kernels that must agree bit for bit do not depend on the compiler's
// contraction choices).
__device__ inline float fma_acc(float a, float b, float c) { return fmaf(a, b, c); }
__device__ inline double fma_acc(double a, double b, double c) { return fma(a, b, c); }

// Four consecutive elements loaded/stored as one vector access. The caller
// guarantees 4-element alignment.
template <typename T, typename Acc>
__device__ inline void load4(const T* __restrict__ p, Acc out[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) out[i] = Cvt<T, Acc>::load(p[i]);
}
template <>
__device__ inline void load4<float, float>(const float* __restrict__ p, float out[4]) {
  float4 v = *reinterpret_cast<const float4*>(p);
  out[0] = v.x;
  out[1] = v.y;
  out[2] = v.z;
  out[3] = v.w;
}
template <>
__device__ inline void load4<bf16_t, float>(const bf16_t* __restrict__ p, float out[4]) {
  uint2 v = *reinterpret_cast<const uint2*>(p);
  out[0] = __uint_as_float(v.x << 16);
  out[1] = __uint_as_float(v.x & 0xffff0000u);
  out[2] = __uint_as_float(v.y << 16);
  out[3] = __uint_as_float(v.y & 0xffff0000u);
}
template <>
__device__ inline void load4<f16_t, float>(const f16_t* __restrict__ p, float out[4]) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  h4 v = *reinterpret_cast<const h4*>(p);
  out[0] = static_cast<float>(v[0]);
  out[1] = static_cast<float>(v[1]);
  out[2] = static_cast<float>(v[2]);
  out[3] = static_cast<float>(v[3]);
}

template <typename T, typename Acc>
__device__ inline void store4(T* __restrict__ p, const Acc in[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = Cvt<T, Acc>::store(in[i]);
}
template <>
__device__ inline void store4<float, float>(float* __restrict__ p, const float in[4]) {
  *reinterpret_cast<float4*>(p) = make_float4(in[0], in[1], in[2], in[3]);
}
template <>
__device__ inline void store4<bf16_t, float>(bf16_t* __restrict__ p, const float in[4]) {
  uint2 v;
  v.x = static_cast<uint32_t>(f32_to_bf16(in[0])) | (static_cast<uint32_t>(f32_to_bf16(in[1])) << 16);
  v.y = static_cast<uint32_t>(f32_to_bf16(in[2])) | (static_cast<uint32_t>(f32_to_bf16(in[3])) << 16);
  *reinterpret_cast<uint2*>(p) = v;
}
template <>
__device__ inline void store4<f16_t, float>(f16_t* __restrict__ p, const float in[4]) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  h4 v;
  v[0] = static_cast<_Float16>(in[0]);
  v[1] = static_cast<_Float16>(in[1]);
  v[2] = static_cast<_Float16>(in[2]);
  v[3] = static_cast<_Float16>(in[3]);
  *reinterpret_cast<h4*>(p) = v;
}

// Eight consecutive elements as 16-byte vector accesses (one for 16-bit
// types, two for fp32, four for fp64). The caller guarantees that the address
// is aligned to 8 elements.
template <typename T, typename Acc>
__device__ inline void load8(const T* __restrict__ p, Acc (&out)[8]) {
  load4<T, Acc>(p, out);
  load4<T, Acc>(p + 4, out + 4);
}
template <>
__device__ inline void load8<bf16_t, float>(const bf16_t* __restrict__ p, float (&out)[8]) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(w[i] << 16);
    out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}
template <>
__device__ inline void load8<f16_t, float>(const f16_t* __restrict__ p, float (&out)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 v = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(v[i]);
}
template <typename T, typename Acc>
__device__ inline void store8(T* __restrict__ p, const Acc (&in)[8]) {
  store4<T, Acc>(p, in);
  store4<T, Acc>(p + 4, in + 4);
}
template <>
__device__ inline void store8<bf16_t, float>(bf16_t* __restrict__ p, const float (&in)[8]) {
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    w[i] = static_cast<uint32_t>(f32_to_bf16(in[2 * i])) | (static_cast<uint32_t>(f32_to_bf16(in[2 * i + 1])) << 16);
  *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
}
template <>
__device__ inline void store8<f16_t, float>(f16_t* __restrict__ p, const float (&in)[8]) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  h8 v;
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<_Float16>(in[i]);
  *reinterpret_cast<h8*>(p) = v;
}

// Element ranges of a row chunk that starts at global element `base` and has
// `len` elements: a scalar head up to the next 8-element boundary, `nvec`
// aligned 8-element vectors, then a scalar tail from `tail0`. Without
// `vec_ok` (tensor pointers not 64-byte aligned) everything is scalar.
struct RowSpan {
  int64_t head, nvec, tail0, len;
  __device__ int64_t scalar_count() const { return head + (len - tail0); }
  __device__ int64_t scalar_index(int64_t i) const { return i < head ? i : tail0 + (i - head); }
};
__device__ inline RowSpan row_span(int64_t base, int64_t len, bool vec_ok) {
  RowSpan s;
  if (len < 0) len = 0;  // a trailing split past the row end is empty
  int64_t h = vec_ok ? ((8 - (base & 7)) & 7) : len;
  if (h > len) h = len;
  s.head = h;
  s.nvec = (len - h) >> 3;
  s.tail0 = h + (s.nvec << 3);
  s.len = len;
  return s;
}

// Wave64 sum via cross-lane shuffles (fixed butterfly order: deterministic).
template <typename Acc>
__device__ inline Acc wave_sum(Acc v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// ---------------------------------------------------------------- host side

void set_error(const std::string& msg);

// Validation helpers used by every entry point. Each returns a C-ABI status.
#define MEDNEXT_CHECK_ARG(cond, msg)                    \
  do {                                                  \
    if (!(cond)) {                                      \
      ::mednext::set_error(std::string(__func__) + ": " + (msg)); \
      return MEDNEXT_STATUS_INVALID_ARGUMENT;           \
    }                                                   \
  } while (0)

#define MEDNEXT_CHECK_LAUNCH()                                                   \
  do {                                                                           \
    hipError_t err_ = hipGetLastError();                                         \
    if (err_ != hipSuccess) {                                                    \
      ::mednext::set_error(std::string(__func__) + ": launch failed: " +        \
                           hipGetErrorString(err_));                              \
      return MEDNEXT_STATUS_LAUNCH_ERROR;                                        \
    }                                                                            \
  } while (0)

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace mednext
