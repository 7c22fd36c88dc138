// gfx950 (CDNA4) device helpers shared by the matrix-core kernels: MFMA
// operand vector types and raw buffer loads/stores.
//
// Raw buffer access: a buffer resource covers [base, base + bytes); a load at
// an offset at or past `bytes` returns zeros and such a store is dropped by the
// hardware, so padding and ragged-edge masking need no branches (kOob is a
// conventional "always out of range" offset). Offsets are 32-bit, so one
// resource spans < 2 GiB.
//
// Lane layout of v_mfma_f32_16x16x32_bf16 (verified on gfx950): lane l holds
// A[l%16][8*(l/16) + j], B[8*(l/16) + j][l%16] (j = 0..7) and
// C[4*(l/16) + r][l%16] (r = 0..3).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace mednext {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));

constexpr uint32_t kOob = 0x80000000u;

__device__ inline __amdgpu_buffer_rsrc_t slab_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), bytes,
                                           0x00020000);
}
// One element through a raw buffer resource; `ok == false` reads the
// out-of-range offset, which returns zero. Keeping every load unconditional
// lets a task issue all of its loads back to back.
template <typename T>
struct BufIo;
template <>
struct BufIo<float> {
  __device__ static float ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  }
  __device__ static void st(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, 0);
  }
};
template <>
struct BufIo<double> {
  __device__ static double ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(double, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
  }
  __device__ static void st(__amdgpu_buffer_rsrc_t r, uint32_t off, double v) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, v), r, off, 0, 0);
  }
};
template <>
struct BufIo<f16_t> {
  __device__ static float ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return static_cast<float>(__builtin_bit_cast(f16_t, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0)));
  }
  __device__ static void st(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, static_cast<f16_t>(v)), r, off, 0, 0);
  }
};
template <>
struct BufIo<bf16_t> {
  __device__ static float ld(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return bf16_to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  }
  __device__ static void st(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(v), r, off, 0, 0);
  }
};

template <typename T>
__device__ inline uint32_t boff(bool ok, int elem) {
  return ok ? static_cast<uint32_t>(elem) * static_cast<uint32_t>(sizeof(T)) : kOob;
}

__device__ inline uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// Streaming load: cache policy 2 sets the non-temporal bit (data read once is
// not kept in the caches). Non-temporal stores measured ~40% slower here.
__device__ inline uint4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ inline uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ inline u32x2_t buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ inline void buf_store2(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, 0);
}
__device__ inline void buf_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}
__device__ inline void buf_store8(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t lo, uint32_t hi) {
  const u32x2_t v = {lo, hi};
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, 0);
}
__device__ inline void buf_store16(__amdgpu_buffer_rsrc_t r, uint32_t off, uint4 v) {
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, r, off, 0, 0);
}

// 8 consecutive bf16 starting at element e of a tensor whose rows have odd
// width, of which the first `valid` are real (the rest read zero). Such rows
// start at any 2-byte boundary, and so may a tensor or slab holding an odd
// number of elements, while multi-byte buffer loads drop the address bits
// below their size: the run is read as eight 2-byte loads (run8_load, issued
// early) and packed once the data is needed (run8_pack).
struct Run8 {
  uint32_t h[8];
};
__device__ inline Run8 run8_load(__amdgpu_buffer_rsrc_t r, uint32_t e, int valid) {
  Run8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o.h[j] = __builtin_amdgcn_raw_buffer_load_b16(r, j < valid ? (e + j) * 2u : kOob, 0, 0);
  return o;
}
__device__ inline uint4 run8_pack(const Run8& p) {
  return make_uint4(p.h[0] | (p.h[1] << 16), p.h[2] | (p.h[3] << 16), p.h[4] | (p.h[5] << 16),
                    p.h[6] | (p.h[7] << 16));
}

// MI355X dispatches workgroup i to XCD i % 8, and each XCD has its own L2.
// Remapping (i % 8, i / 8) -> (i % 8) * (n / 8) + i / 8 hands every XCD a
// contiguous run of tile indices, so neighbouring tiles (which share halo
// cache lines) meet in one L2. Bijective on [0, 8 * (n / 8)); the < 8 tail
// keeps its index.
constexpr int kXcds = 8;
__device__ inline int64_t xcd_swizzle(int64_t bid, int64_t nblocks) {
  const int64_t per = nblocks / kXcds;
  if (bid >= per * kXcds) return bid;
  return (bid % kXcds) * per + bid / kXcds;
}

__device__ inline f32x4_t mfma16x16x32(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// Two floats -> packed bf16 pair (round to nearest even), low half = a.
__device__ inline uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ inline float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ inline float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

}  // namespace mednext
