// Band kernels: depthwise Conv3d on small planes (stride 1) and the stride-2
// down / up maps, every dtype; fp32 accumulation (fp64 for fp64).
//
// Stride 1, small planes (H * W <= 256: the MedNeXt stages at 16^3 and 8^3).
// The tiled kernels leave most lanes idle at these sizes (a 16 x 16 plane is
// one or two column tiles) and run long serial per-thread chains, so they are
// latency-bound at 30-60 us for 1-4 MB of data. Here the work is cut so that
// every lane runs a short chain of useful FMAs:
//
// A workgroup owns one (n, c) slab, one band of kBand = 64 consecutive plane
// positions (row-major (h, w): a 16 x 16 plane has four bands of four rows,
// an 8 x 8 plane one) and one D-run of TD output planes. It has k waves:
// wave kh takes kernel row kh, lane l the band's position l. The zero-padded
// input rows the band needs (its rows plus P above and below, W + 2P columns)
// of the TD + 2P planes the D-run reaches are staged once in LDS, converted
// to the accumulation type.
//
// Each lane walks the staged planes front to back. Per input plane it reads
// the k values of its kernel row (x[pd][h + kh][w .. w + k - 1]) and applies
// them to every tap along D, k * k FMAs:
//   forward / input gradient: into a register ring of the k output planes the
//     input plane reaches, with this kernel row's k * k weights in registers.
//     An output plane leaves the ring complete for the row and goes to LDS;
//     the k rows' sums (+ bias) are then added in a fixed order and stored,
//     one contiguous 64-position run per plane;
//   weight gradient: against a register ring of the k most recent
//     grad_output values (staged in LDS with the input), into the row's k * k
//     tap sums and the bias sum. The lane sums are reduced per wave in a
//     fixed order through LDS (16-lane segments, then the four segments) into
//     the same [C][k^3 + 1][splits] partial layout as the other
//     weight-gradient kernels; the shared fixed-order finish kernel sums the
//     splits.
// The first and last k - 1 planes of the walk are unrolled with only the taps
// whose output (forward) or grad_output (weight gradient) plane exists in the
// D-run, so no FMA is spent on the zero padding along D.
//
// Stride 2 (the down block's conv, padding k/2, and the up block's transposed
// conv), between a full-resolution "big" and a half-resolution "small" tensor:
//   gather  small[o] = b + sum_t w[t] big[2o + t - P]
//   reduce  dW[t] = sum_o big[2o + t - P] small[o], dB = sum_o small[o]
// The same decomposition over the SMALL plane: a workgroup owns a band of 64
// small positions and a D-run of TD small planes, and stages the big rows and
// planes they reach (rows 2 hs - P .. 2 hs + P of each small row hs, planes
// 2 d - P .. 2 d + P of each small plane d). Lane (kh, small position (hs,
// ws)) reads big row 2 (hs - hs0) + kh, columns 2 ws .. 2 ws + k - 1 of each
// staged plane. Big plane 2m + e (e in {0, 1}) meets small plane m - i
// through tap kd = 2i + e, so the walk goes in plane pairs with a register
// ring of P + 1 small planes (outputs for the gather, grad_output /
// input values for the reduce). A reduce workgroup walks several bands of one
// (slab, D-run) before its single reduction, which keeps the partials few.
#include "cdna4.h"
#include "common.h"
#include "depthwise_volume.h"

#include <algorithm>

namespace mednext {
namespace {

constexpr int kBand = 64;       // plane positions per workgroup: one wave's lanes
constexpr int kFillBatch = 8;   // element loads in flight per thread while staging
constexpr int kChunkBatch = 4;  // 4-element chunk loads in flight per thread while staging
constexpr int kDyBatch = 4;     // band-vector loads in flight per thread

// A block of zero-padded rows staged in LDS: rows [row0, row0 + rows) x
// columns [-P, W + P) of planes [plane0, plane0 + planes) of one D x H x W
// slab, stored lds[plane][row][col] (row pitch W + 2P), zero outside the slab.
struct StageGeom {
  int D, H, W;
  int rows, planes;
  uint32_t wp_magic;     // ceil(2^31 / (W + 2P))
  uint32_t plane_magic;  // ceil(2^31 / (rows * (W + 2P)))
  uint32_t w4_magic;     // ceil(2^31 / (W / 4)) (W % 4 == 0 only)
  uint32_t rows_magic;   // ceil(2^31 / rows)
};

// n / d for n * d < 2^31 with magic = ceil(2^31 / d): n * magic / 2^31 exceeds
// n / d by less than n / 2^31 < 1 / d, which never reaches the next integer.
__device__ inline int div_magic(int n, uint32_t magic) {
  return static_cast<int>(__umulhi(static_cast<uint32_t>(n) << 1, magic));
}

template <typename T, typename Acc>
__device__ inline Acc load_acc(const T* p, int64_t i) {
  return Cvt<T, Acc>::load(p[i]);
}

// Four consecutive elements through a raw buffer resource (one 8-byte load
// for 16-bit types), converted to the accumulation type; the out-of-range
// offset reads zeros.
template <typename T>
struct BufIo4;
template <>
struct BufIo4<bf16_t> {
  __device__ static void ld(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[4]) {
    const u32x2_t q = buf_load8(r, off);
    v[0] = bf16_to_f32(static_cast<uint16_t>(q[0]));
    v[1] = bf16_to_f32(static_cast<uint16_t>(q[0] >> 16));
    v[2] = bf16_to_f32(static_cast<uint16_t>(q[1]));
    v[3] = bf16_to_f32(static_cast<uint16_t>(q[1] >> 16));
  }
};
template <>
struct BufIo4<f16_t> {
  __device__ static void ld(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[4]) {
    const u32x2_t q = buf_load8(r, off);
    v[0] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(q[0])));
    v[1] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(q[0] >> 16)));
    v[2] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(q[1])));
    v[3] = static_cast<float>(__builtin_bit_cast(f16_t, static_cast<uint16_t>(q[1] >> 16)));
  }
};
template <>
struct BufIo4<float> {
  __device__ static void ld(__amdgpu_buffer_rsrc_t r, uint32_t off, float (&v)[4]) {
    const uint4 q = buf_load16(r, off);
    v[0] = __uint_as_float(q.x);
    v[1] = __uint_as_float(q.y);
    v[2] = __uint_as_float(q.z);
    v[3] = __uint_as_float(q.w);
  }
};
template <>
struct BufIo4<double> {
  __device__ static void ld(__amdgpu_buffer_rsrc_t r, uint32_t off, double (&v)[4]) {
    const uint4 a = buf_load16(r, off);
    const uint4 b = buf_load16(r, off == kOob ? kOob : off + 16);
    v[0] = __hiloint2double(a.y, a.x);
    v[1] = __hiloint2double(a.w, a.z);
    v[2] = __hiloint2double(b.y, b.x);
    v[3] = __hiloint2double(b.w, b.z);
  }
};

template <typename T>
__device__ inline __amdgpu_buffer_rsrc_t slab_buffer(const T* slab, int64_t elems) {
  return slab_rsrc(slab, static_cast<uint32_t>(elems * static_cast<int64_t>(sizeof(T))));
}

// Element-wise staging. Consecutive threads take consecutive columns of a row;
// loads go through a raw buffer resource over the slab and out-of-slab
// elements read the out-of-range offset (zero), so each thread issues
// kFillBatch loads back to back with no branches before its first store.
template <typename T, typename Acc, int P>
__device__ inline void stage_rows_scalar(Acc* __restrict__ lds, const T* __restrict__ slab, const StageGeom& s,
                                         int plane0, int row0, int nthreads) {
  const int Wp = s.W + 2 * P;
  const int per_plane = s.rows * Wp;
  const int total = s.planes * per_plane;
  const int plane = s.H * s.W;
  const __amdgpu_buffer_rsrc_t src = slab_buffer(slab, static_cast<int64_t>(s.D) * plane);
  for (int base = 0; base < total; base += nthreads * kFillBatch) {
    Acc v[kFillBatch];
#pragma unroll
    for (int b = 0; b < kFillBatch; ++b) {
      v[b] = Acc(0);
      if (base + b * nthreads >= total) break;  // uniform: no load for slots past the staged block
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      const int pd = div_magic(e, s.plane_magic);
      const int r = e - pd * per_plane;
      const int sr = div_magic(r, s.wp_magic);
      const int gw = r - sr * Wp - P;
      const int gh = row0 + sr;
      const int gd = plane0 + pd;
      const bool ok = e < total && gd >= 0 && gd < s.D && gh >= 0 && gh < s.H && gw >= 0 && gw < s.W;
      v[b] = BufIo<T>::ld(src, boff<T>(ok, gd * plane + gh * s.W + gw));
    }
#pragma unroll
    for (int b = 0; b < kFillBatch; ++b) {
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      if (e < total) lds[e] = v[b];
    }
  }
}

// W % 4 == 0: the interior of each staged row is loaded in 4-column chunks (a
// quarter of the load instructions and index arithmetic), and the 2P padding
// columns of every row are written as zeros.
template <typename T, typename Acc, int P, int CB>
__device__ inline void stage_rows_w4(Acc* __restrict__ lds, const T* __restrict__ slab, const StageGeom& s,
                                     int plane0, int row0, int nthreads) {
  const int Wp = s.W + 2 * P, W4 = s.W >> 2;
  const int rows = s.planes * s.rows;
  const int total = rows * W4;
  const int plane = s.H * s.W;
  const __amdgpu_buffer_rsrc_t src = slab_buffer(slab, static_cast<int64_t>(s.D) * plane);
  for (int base = 0; base < total; base += nthreads * CB) {
    Acc v[CB][4];
    int dst[CB];  // LDS element offset of the chunk, -1: nothing to store
#pragma unroll
    for (int b = 0; b < CB; ++b) dst[b] = -1;
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      if (base + b * nthreads >= total) break;  // uniform
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      const int row = div_magic(e, s.w4_magic);
      const int cx = e - row * W4;
      const int pd = div_magic(row, s.rows_magic);
      const int sr = row - pd * s.rows;
      const int gh = row0 + sr;
      const int gd = plane0 + pd;
      const bool ok = e < total && gd >= 0 && gd < s.D && gh >= 0 && gh < s.H;
      BufIo4<T>::ld(src, boff<T>(ok, gd * plane + gh * s.W + 4 * cx), v[b]);
      dst[b] = e < total ? row * Wp + P + 4 * cx : -1;
    }
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      if (dst[b] >= 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) lds[dst[b] + j] = v[b][j];
      }
    }
  }
  if (P > 0) {
    for (int row = threadIdx.x; row < rows; row += nthreads) {
#pragma unroll
      for (int j = 0; j < P; ++j) {
        lds[row * Wp + j] = Acc(0);
        lds[row * Wp + P + s.W + j] = Acc(0);
      }
    }
  }
}

template <typename T, typename Acc, int P, int CB = kChunkBatch>
__device__ inline void stage_rows(Acc* __restrict__ lds, const T* __restrict__ slab, const StageGeom& s, int plane0,
                                  int row0, int nthreads) {
  if ((s.W & 3) == 0)
    stage_rows_w4<T, Acc, P, CB>(lds, slab, s, plane0, row0, nthreads);
  else
    stage_rows_scalar<T, Acc, P>(lds, slab, s, plane0, row0, nthreads);
}

// A band's vector: ds[od][l] = v[(d0 + od) * hw + p0 + l] of one slab for
// od < nd, l < nb, zero elsewhere in [0, walk) x [0, kBand); CW consecutive
// positions per load (CW = 4 needs hw % 4 == 0).
struct BandVec {
  int D, hw, d0, nd, p0, nb, walk;
};

template <typename T, typename Acc, int CW>
__device__ inline void band_vec_load(Acc (&v)[kDyBatch][CW], __amdgpu_buffer_rsrc_t src, const BandVec& b,
                                     int base, int nthreads) {
  constexpr int per_plane = kBand / CW;
  const int total = b.walk * per_plane;
#pragma unroll
  for (int i = 0; i < kDyBatch; ++i) {
    const int e = base + i * nthreads + static_cast<int>(threadIdx.x);
    const int od = e / per_plane, l = (e % per_plane) * CW;
    const uint32_t off = boff<T>(e < total && od < b.nd && l < b.nb, (b.d0 + od) * b.hw + b.p0 + l);
    if constexpr (CW == 4) {
      BufIo4<T>::ld(src, off, v[i]);
    } else {
      v[i][0] = BufIo<T>::ld(src, off);
    }
  }
}

template <typename Acc, int CW>
__device__ inline void band_vec_store(Acc* __restrict__ ds, const Acc (&v)[kDyBatch][CW], const BandVec& b, int base,
                                      int nthreads) {
  constexpr int per_plane = kBand / CW;
  const int total = b.walk * per_plane;
#pragma unroll
  for (int i = 0; i < kDyBatch; ++i) {
    const int e = base + i * nthreads + static_cast<int>(threadIdx.x);
    if (e < total) {
#pragma unroll
      for (int j = 0; j < CW; ++j) ds[(e / per_plane) * kBand + (e % per_plane) * CW + j] = v[i][j];
    }
  }
}

// The weight gradients' staging: the band vector's first batch of loads is
// issued before the rows are staged and stays in flight meanwhile.
template <typename T, typename Acc, int P, int CW, int CB>
__device__ inline void stage_rows_and_vec_cw(Acc* __restrict__ xs, Acc* __restrict__ ds, const T* __restrict__ xslab,
                                             const StageGeom& s, int plane0, int row0, const T* __restrict__ vslab,
                                             const BandVec& b, int nthreads) {
  const __amdgpu_buffer_rsrc_t src = slab_buffer(vslab, static_cast<int64_t>(b.D) * b.hw);
  const int total = b.walk * (kBand / CW);
  Acc v[kDyBatch][CW];
  band_vec_load<T, Acc, CW>(v, src, b, 0, nthreads);
  stage_rows<T, Acc, P, CB>(xs, xslab, s, plane0, row0, nthreads);
  band_vec_store<Acc, CW>(ds, v, b, 0, nthreads);
  for (int base = nthreads * kDyBatch; base < total; base += nthreads * kDyBatch) {
    band_vec_load<T, Acc, CW>(v, src, b, base, nthreads);
    band_vec_store<Acc, CW>(ds, v, b, base, nthreads);
  }
}

template <typename T, typename Acc, int P, int CB = kChunkBatch>
__device__ inline void stage_rows_and_vec(Acc* __restrict__ xs, Acc* __restrict__ ds, const T* __restrict__ xslab,
                                          const StageGeom& s, int plane0, int row0, const T* __restrict__ vslab,
                                          const BandVec& b, int nthreads) {
  if ((b.hw & 3) == 0)
    stage_rows_and_vec_cw<T, Acc, P, 4, CB>(xs, ds, xslab, s, plane0, row0, vslab, b, nthreads);
  else
    stage_rows_and_vec_cw<T, Acc, P, 1, CB>(xs, ds, xslab, s, plane0, row0, vslab, b, nthreads);
}

template <typename Acc, int K>
__device__ inline void load_row(Acc (&xv)[K], const Acc* __restrict__ p) {
#pragma unroll
  for (int kw = 0; kw < K; ++kw) xv[kw] = p[kw];
}

template <typename Acc, int N>
__device__ inline void shift_ring(Acc (&ring)[N]) {
#pragma unroll
  for (int j = N - 1; j > 0; --j) ring[j] = ring[j - 1];
}

// Values per lane (one kernel row's taps + the bias sum) reduced per LDS
// round: all of them, except fp64 at k = 5, whose 26 values per lane are
// reduced in two rounds to stay within the staged LDS footprint.
template <typename Acc, int K>
constexpr int band_red_values() {
  return sizeof(Acc) == 8 && K == 5 ? 13 : K * K + 1;
}

// Per-wave fixed-order reduction over the 64 lanes of wave kh's k * k tap
// sums acc[kd][kw] (+ the bias sum, kept from wave 0 only), through LDS that
// aliases the staged planes (value r0 + i of lane l at red[l * PITCH + i]),
// into partial[(c * (k^3 + 1) + tap) * splits + split]. Every wave calls it.
template <typename Acc, int K>
__device__ inline void reduce_row_taps(const Acc (&acc)[K][K], Acc bsum, Acc* __restrict__ lds, int kh, int lane,
                                       Acc* __restrict__ partial, int64_t c, int splits, int64_t split) {
  constexpr int K2 = K * K, K3 = K2 * K;
  constexpr int NACC = K2 + 1;
  constexpr int RT = band_red_values<Acc, K>();
  constexpr int PITCH = RT | 1;  // odd: lane-strided LDS accesses hit distinct banks
  Acc* __restrict__ red = lds + kh * kBand * PITCH;
#pragma unroll
  for (int r0 = 0; r0 < NACC; r0 += RT) {
    __syncthreads();  // staged planes (first round) / previous round read by every wave
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int v = r0 + i;
      if (v < NACC) red[lane * PITCH + i] = v < K2 ? acc[v / K][v % K] : bsum;
    }
    __syncthreads();
    const int nr = min(RT, NACC - r0);
    // Item j = (value i, 16-lane segment q); the four segments of a value sit
    // in one lane quad and are added with two butterflies.
    for (int j0 = 0; j0 < nr * 4; j0 += kBand) {
      const int j = j0 + lane;
      const int i = j >> 2, q = j & 3;
      Acc s = Acc(0);
      if (j < nr * 4) {
#pragma unroll
        for (int l = 0; l < 16; ++l) s += red[(q * 16 + l) * PITCH + i];
      }
      s += __shfl_xor(s, 1);
      s += __shfl_xor(s, 2);
      const int v = r0 + i;
      if (j < nr * 4 && q == 0 && (v < K2 || kh == 0)) {
        const int tap = v < K2 ? ((v / K) * K + kh) * K + v % K : K3;
        partial[(c * (K3 + 1) + tap) * splits + split] = s;
      }
    }
  }
}

template <typename Acc, int K>
__host__ __device__ constexpr int band_red_pitch() {
  return band_red_values<Acc, K>() | 1;
}

// ------------------------------------------------------------------ stride 1

struct BandGeom {
  int C, D, H, W;
  int TD;      // output planes per D-run
  int TDk;     // planes the lanes walk: max(TD, k - 1); planes past the D-run are zero / not stored
  int nDc;     // D-runs per slab
  int nbands;  // bands per plane
  StageGeom sg;  // rows = the most rows a band spans + 2P, planes = TDk + 2P
  int64_t slabs;
};

// Workgroup -> (slab, band, D-run); the D-run varies fastest.
struct BandTile {
  int64_t slab;
  int band, dc, d0, nd, p0, hb0;
};

__device__ inline BandTile band_tile(const BandGeom& g) {
  BandTile t;
  t.dc = static_cast<int>(blockIdx.x % g.nDc);
  const int rest = static_cast<int>(blockIdx.x / g.nDc);
  t.band = rest % g.nbands;
  t.slab = rest / g.nbands;
  t.d0 = t.dc * g.TD;
  t.nd = min(g.TD, g.D - t.d0);
  t.p0 = t.band * kBand;
  t.hb0 = t.p0 / g.W;
  return t;
}

template <typename T, typename Acc, int K, bool FLIP, bool BIAS>
__global__ __launch_bounds__(kBand * K) void dw_band_stencil_kernel(const T* __restrict__ x,
                                                                    const T* __restrict__ wt,
                                                                    const T* __restrict__ bias,
                                                                    T* __restrict__ y, BandGeom g) {
  constexpr int P = K / 2, K3 = K * K * K, NT = kBand * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Wp = g.W + 2 * P;
  const int per_plane = g.sg.rows * Wp;
  Acc* const rows = xs + g.sg.planes * per_plane;  // [K][TDk][kBand] per-kernel-row sums
  const int hw = g.H * g.W;

  const BandTile t = band_tile(g);
  stage_rows<T, Acc, P>(xs, x + t.slab * g.D * hw, g.sg, t.d0 - P, t.hb0 - P, NT);

  // Wave kh holds the k * k taps of kernel row kh (flipped for the input gradient).
  const int kh = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kBand);
  const int lane = static_cast<int>(threadIdx.x) % kBand;
  const int64_t c = t.slab % g.C;
  Acc wr[K][K];
#pragma unroll
  for (int kd = 0; kd < K; ++kd)
#pragma unroll
    for (int kw = 0; kw < K; ++kw) {
      const int tap = (kd * K + kh) * K + kw;
      wr[kd][kw] = load_acc<T, Acc>(wt, c * K3 + (FLIP ? K3 - 1 - tap : tap));
    }
  __syncthreads();

  // Lanes past the plane walk its last position and store nothing.
  const int pos = min(t.p0 + lane, hw - 1);
  const int h = pos / g.W, w = pos - h * g.W;
  const Acc* __restrict__ xr = xs + (h - t.hb0 + kh) * Wp + w;
  Acc* __restrict__ rr = rows + kh * g.TDk * kBand + lane;

  // ring[j] = this row's sum for output plane pd - j.
  Acc ring[K];
#pragma unroll
  for (int j = 0; j < K; ++j) ring[j] = Acc(0);
  Acc xv[K];
  // Planes 0 .. K-2: outputs pd - kd < 0 do not exist.
#pragma unroll
  for (int pd = 0; pd < K - 1; ++pd) {
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = 0; kd <= pd; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[kd] += wr[kd][kw] * xv[kw];
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  for (int pd = K - 1; pd < g.TDk; ++pd) {
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = 0; kd < K; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[kd] += wr[kd][kw] * xv[kw];
    rr[(pd - (K - 1)) * kBand] = ring[K - 1];
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  // Planes TDk .. TDk+K-2: outputs pd - kd >= TDk do not exist.
#pragma unroll
  for (int q = 0; q < K - 1; ++q) {
    const int pd = g.TDk + q;
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = q + 1; kd < K; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[kd] += wr[kd][kw] * xv[kw];
    rr[(pd - (K - 1)) * kBand] = ring[K - 1];
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  __syncthreads();

  // Output = bias + row 0 + ... + row K-1, one 64-position run per plane.
  const Acc b = BIAS ? load_acc<T, Acc>(bias, c) : Acc(0);
  const int nb = min(kBand, hw - t.p0);
  T* __restrict__ out = y + (t.slab * g.D + t.d0) * hw + t.p0;
  for (int e = threadIdx.x; e < t.nd * kBand; e += NT) {
    const int od = e / kBand, l = e % kBand;
    if (l >= nb) continue;
    Acc v = b;
#pragma unroll
    for (int r = 0; r < K; ++r) v += rows[(r * g.TDk + od) * kBand + l];
    out[static_cast<int64_t>(od) * hw + l] = Cvt<T, Acc>::store(v);
  }
}

template <typename T, typename Acc, int K>
__global__ __launch_bounds__(kBand * K) void dw_band_wgrad_kernel(const T* __restrict__ x,
                                                                  const T* __restrict__ dy,
                                                                  Acc* __restrict__ partial, BandGeom g,
                                                                  int splits) {
  constexpr int P = K / 2, NT = kBand * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Wp = g.W + 2 * P;
  const int per_plane = g.sg.rows * Wp;
  Acc* const ds = xs + g.sg.planes * per_plane;  // [TDk][kBand] grad_output of the band
  const int hw = g.H * g.W;

  const BandTile t = band_tile(g);
  const BandVec bv{g.D, hw, t.d0, t.nd, t.p0, min(kBand, hw - t.p0), g.TDk};
  const int64_t slab_off = t.slab * g.D * hw;
  stage_rows_and_vec<T, Acc, P>(xs, ds, x + slab_off, g.sg, t.d0 - P, t.hb0 - P, dy + slab_off, bv, NT);
  __syncthreads();

  const int kh = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kBand);
  const int lane = static_cast<int>(threadIdx.x) % kBand;
  // Lanes past the plane walk its last position against zero grad_output.
  const int pos = min(t.p0 + lane, hw - 1);
  const int h = pos / g.W, w = pos - h * g.W;
  const Acc* __restrict__ xr = xs + (h - t.hb0 + kh) * Wp + w;
  const Acc* __restrict__ dr = ds + lane;

  Acc acc[K][K];
#pragma unroll
  for (int kd = 0; kd < K; ++kd)
#pragma unroll
    for (int kw = 0; kw < K; ++kw) acc[kd][kw] = Acc(0);
  Acc bsum = Acc(0);
  Acc ring[K];  // ring[j] = grad_output plane pd - j
#pragma unroll
  for (int j = 0; j < K; ++j) ring[j] = Acc(0);
  Acc xv[K];
  // Input plane pd meets grad_output plane pd - kd through tap kd; planes
  // 0 .. K-2 have no grad_output plane pd - kd < 0.
#pragma unroll
  for (int pd = 0; pd < K - 1; ++pd) {
    shift_ring(ring);
    ring[0] = dr[pd * kBand];
    bsum += ring[0];
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = 0; kd <= pd; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) acc[kd][kw] += xv[kw] * ring[kd];
  }
  for (int pd = K - 1; pd < g.TDk; ++pd) {
    shift_ring(ring);
    ring[0] = dr[pd * kBand];
    bsum += ring[0];
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = 0; kd < K; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) acc[kd][kw] += xv[kw] * ring[kd];
  }
  // Planes TDk .. TDk+K-2 have no grad_output plane pd - kd >= TDk.
#pragma unroll
  for (int q = 0; q < K - 1; ++q) {
    const int pd = g.TDk + q;
    shift_ring(ring);
    ring[0] = Acc(0);
    load_row(xv, xr + pd * per_plane);
#pragma unroll
    for (int kd = q + 1; kd < K; ++kd)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) acc[kd][kw] += xv[kw] * ring[kd];
  }

  const int64_t c = t.slab % g.C, n = t.slab / g.C;
  const int64_t split = (n * g.nbands + t.band) * g.nDc + t.dc;
  reduce_row_taps<Acc, K>(acc, bsum, xs, kh, lane, partial, c, splits, split);
}

// ------------------------------------------------------------------ stride 2

struct S2BandGeom {
  int C;
  int Db, Hb, Wb;  // big
  int Ds, Hs, Ws;  // small
  int TD;          // small planes per D-run
  int TDk;         // small planes walked: max(TD, P)
  int nDc;         // D-runs per slab
  int nbands;      // bands of kBand small positions per small plane
  int bpw;         // bands one reduce workgroup walks
  int nbw;         // reduce workgroups per (slab, D-run): ceil(nbands / bpw)
  StageGeom sg;    // big rows 2 hs0 - P + [0, rows), planes 2 d0 - P + [0, 2 TDk + k - 2)
  int64_t slabs;
};

template <typename T, typename Acc, int K, bool BIAS>
__global__ __launch_bounds__(kBand * K) void dw_s2band_gather_kernel(const T* __restrict__ big,
                                                                     const T* __restrict__ wt,
                                                                     const T* __restrict__ bias,
                                                                     T* __restrict__ small, S2BandGeom g) {
  constexpr int P = K / 2, K3 = K * K * K, NT = kBand * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Wp = g.Wb + 2 * P;
  const int per_plane = g.sg.rows * Wp;
  Acc* const rows = xs + g.sg.planes * per_plane;  // [K][TDk][kBand] per-kernel-row sums
  const int hws = g.Hs * g.Ws;

  const int dc = static_cast<int>(blockIdx.x % g.nDc);
  const int rest = static_cast<int>(blockIdx.x / g.nDc);
  const int band = rest % g.nbands;
  const int64_t slab = rest / g.nbands;
  const int d0 = dc * g.TD, nd = min(g.TD, g.Ds - d0);
  const int p0 = band * kBand, hs0 = p0 / g.Ws;
  stage_rows<T, Acc, P>(xs, big + slab * g.Db * g.Hb * g.Wb, g.sg, 2 * d0 - P, 2 * hs0 - P, NT);

  const int kh = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kBand);
  const int lane = static_cast<int>(threadIdx.x) % kBand;
  const int64_t c = slab % g.C;
  Acc wr[K][K];
#pragma unroll
  for (int kd = 0; kd < K; ++kd)
#pragma unroll
    for (int kw = 0; kw < K; ++kw) wr[kd][kw] = load_acc<T, Acc>(wt, c * K3 + (kd * K + kh) * K + kw);
  __syncthreads();

  const int pos = min(p0 + lane, hws - 1);
  const int hs = pos / g.Ws, ws = pos - hs * g.Ws;
  const Acc* __restrict__ xr = xs + (2 * (hs - hs0) + kh) * Wp + 2 * ws;
  Acc* __restrict__ rr = rows + kh * g.TDk * kBand + lane;

  // Pair m: big plane 2m + e meets output m - i through tap kd = 2i + e.
  // ring[i] = this row's sum for output m - i.
  Acc ring[P + 1];
#pragma unroll
  for (int i = 0; i <= P; ++i) ring[i] = Acc(0);
  Acc xv[K];
  // Pairs 0 .. P-1: outputs m - i < 0 do not exist.
#pragma unroll
  for (int m = 0; m < P; ++m) {
    load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
    for (int i = 0; i <= m; ++i)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i][kw] * xv[kw];
    load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
    for (int i = 0; i <= m && i < P; ++i)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i + 1][kw] * xv[kw];
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  for (int m = P; m < g.TDk; ++m) {
    load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
    for (int i = 0; i <= P; ++i)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i][kw] * xv[kw];
    rr[(m - P) * kBand] = ring[P];
    if constexpr (P > 0) {
      load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
      for (int i = 0; i < P; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i + 1][kw] * xv[kw];
    }
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  // Pairs TDk .. TDk+P-1: outputs m - i >= TDk do not exist.
#pragma unroll
  for (int q = 0; q < P; ++q) {
    const int m = g.TDk + q;
    load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
    for (int i = q + 1; i <= P; ++i)
#pragma unroll
      for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i][kw] * xv[kw];
    rr[(m - P) * kBand] = ring[P];
    if (q + 1 < P) {
      load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
      for (int i = q + 1; i < P; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) ring[i] += wr[2 * i + 1][kw] * xv[kw];
    }
    shift_ring(ring);
    ring[0] = Acc(0);
  }
  __syncthreads();

  const Acc b = BIAS ? load_acc<T, Acc>(bias, c) : Acc(0);
  const int nb = min(kBand, hws - p0);
  T* __restrict__ out = small + (slab * g.Ds + d0) * hws + p0;
  for (int e = threadIdx.x; e < nd * kBand; e += NT) {
    const int od = e / kBand, l = e % kBand;
    if (l >= nb) continue;
    Acc v = b;
#pragma unroll
    for (int r = 0; r < K; ++r) v += rows[(r * g.TDk + od) * kBand + l];
    out[static_cast<int64_t>(od) * hws + l] = Cvt<T, Acc>::store(v);
  }
}

template <typename T, typename Acc, int K>
__global__ __launch_bounds__(kBand * K) void dw_s2band_wgrad_kernel(const T* __restrict__ big,
                                                                    const T* __restrict__ small,
                                                                    Acc* __restrict__ partial, S2BandGeom g,
                                                                    int splits) {
  constexpr int P = K / 2, NT = kBand * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Wp = g.Wb + 2 * P;
  const int per_plane = g.sg.rows * Wp;
  Acc* const ds = xs + g.sg.planes * per_plane;  // [TDk][kBand] small values of the band
  const int hws = g.Hs * g.Ws;

  const int dc = static_cast<int>(blockIdx.x % g.nDc);
  const int rest = static_cast<int>(blockIdx.x / g.nDc);
  const int bg = rest % g.nbw;
  const int64_t slab = rest / g.nbw;
  const int d0 = dc * g.TD, nd = min(g.TD, g.Ds - d0);
  const T* __restrict__ bslab = big + slab * g.Db * g.Hb * g.Wb;
  const T* __restrict__ sslab = small + slab * g.Ds * hws;
  const int kh = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / kBand);
  const int lane = static_cast<int>(threadIdx.x) % kBand;
  const Acc* __restrict__ dr = ds + lane;

  Acc acc[K][K];
#pragma unroll
  for (int kd = 0; kd < K; ++kd)
#pragma unroll
    for (int kw = 0; kw < K; ++kw) acc[kd][kw] = Acc(0);
  Acc bsum = Acc(0);
  const int band_end = min((bg + 1) * g.bpw, g.nbands);
  for (int band = bg * g.bpw; band < band_end; ++band) {
    const int p0 = band * kBand, hs0 = p0 / g.Ws;
    const BandVec bv{g.Ds, hws, d0, nd, p0, min(kBand, hws - p0), g.TDk};
    __syncthreads();  // the previous band's planes are read by every wave
    stage_rows_and_vec<T, Acc, P>(xs, ds, bslab, g.sg, 2 * d0 - P, 2 * hs0 - P, sslab, bv, NT);
    __syncthreads();
    // Lanes past the plane walk its last position against zero small values.
    const int pos = min(p0 + lane, hws - 1);
    const int hs = pos / g.Ws, ws = pos - hs * g.Ws;
    const Acc* __restrict__ xr = xs + (2 * (hs - hs0) + kh) * Wp + 2 * ws;
    // Pair m: big plane 2m + e meets small plane m - i through tap kd = 2i + e.
    Acc ring[P + 1];  // ring[i] = small plane m - i
#pragma unroll
    for (int i = 0; i <= P; ++i) ring[i] = Acc(0);
    Acc xv[K];
#pragma unroll
    for (int m = 0; m < P; ++m) {
      shift_ring(ring);
      ring[0] = dr[m * kBand];
      bsum += ring[0];
      load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
      for (int i = 0; i <= m; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) acc[2 * i][kw] += xv[kw] * ring[i];
      load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
      for (int i = 0; i <= m && i < P; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) acc[2 * i + 1][kw] += xv[kw] * ring[i];
    }
    for (int m = P; m < g.TDk; ++m) {
      shift_ring(ring);
      ring[0] = dr[m * kBand];
      bsum += ring[0];
      load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
      for (int i = 0; i <= P; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) acc[2 * i][kw] += xv[kw] * ring[i];
      if constexpr (P > 0) {
        load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
        for (int i = 0; i < P; ++i)
#pragma unroll
          for (int kw = 0; kw < K; ++kw) acc[2 * i + 1][kw] += xv[kw] * ring[i];
      }
    }
#pragma unroll
    for (int q = 0; q < P; ++q) {
      const int m = g.TDk + q;
      shift_ring(ring);
      ring[0] = Acc(0);
      load_row(xv, xr + 2 * m * per_plane);
#pragma unroll
      for (int i = q + 1; i <= P; ++i)
#pragma unroll
        for (int kw = 0; kw < K; ++kw) acc[2 * i][kw] += xv[kw] * ring[i];
      if (q + 1 < P) {
        load_row(xv, xr + (2 * m + 1) * per_plane);
#pragma unroll
        for (int i = q + 1; i < P; ++i)
#pragma unroll
          for (int kw = 0; kw < K; ++kw) acc[2 * i + 1][kw] += xv[kw] * ring[i];
      }
    }
  }

  const int64_t c = slab % g.C, n = slab / g.C;
  const int64_t split = (n * g.nbw + bg) * g.nDc + dc;
  reduce_row_taps<Acc, K>(acc, bsum, xs, kh, lane, partial, c, splits, split);
}

// ------------------------------------------------------------------ host

// The most plane rows one band of kBand positions of an h x w plane spans.
int64_t band_rows(int64_t h, int64_t w) {
  const int64_t hw = h * w;
  int64_t most = 1;
  for (int64_t p0 = 0; p0 < hw; p0 += kBand) {
    const int64_t last = std::min<int64_t>(p0 + kBand, hw) - 1;
    most = std::max<int64_t>(most, last / w - p0 / w + 1);
  }
  return most;
}

uint32_t magic31(int64_t d) { return static_cast<uint32_t>(((int64_t(1) << 31) + d - 1) / d); }

StageGeom make_stage(int64_t d, int64_t h, int64_t w, int rows, int planes, int P) {
  StageGeom s{};
  s.D = static_cast<int>(d);
  s.H = static_cast<int>(h);
  s.W = static_cast<int>(w);
  s.rows = rows;
  s.planes = planes;
  s.wp_magic = magic31(w + 2 * P);
  s.plane_magic = magic31(static_cast<int64_t>(rows) * (w + 2 * P));
  s.w4_magic = magic31(std::max<int64_t>(1, w / 4));
  s.rows_magic = magic31(rows);
  return s;
}

size_t staged_elems(const StageGeom& s, int P) { return static_cast<size_t>(s.planes) * s.rows * (s.W + 2 * P); }

size_t red_elems(int k, int acc_bytes) {
  const int rt = acc_bytes == 8 && k == 5 ? 13 : k * k + 1;
  return static_cast<size_t>(k) * kBand * (rt | 1);
}

int64_t elem_bytes(int dtype) { return dtype == MEDNEXT_DTYPE_F64 ? 8 : dtype == MEDNEXT_DTYPE_F32 ? 4 : 2; }

size_t band_lds_bytes(const BandGeom& g, int k, int acc_bytes, bool wgrad) {
  const size_t staged = staged_elems(g.sg, k / 2);
  if (!wgrad) return (staged + static_cast<size_t>(k) * g.TDk * kBand) * acc_bytes;
  return std::max(staged + static_cast<size_t>(g.TDk) * kBand, red_elems(k, acc_bytes)) * acc_bytes;
}

int band_plan(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int band, int depth_chunk,
              bool wgrad, BandGeom* g, size_t* lds) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h >= 1 && w >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  MEDNEXT_CHECK_ARG(h * w <= 4 * kBand, "the volume engine takes planes of at most 256 elements (H * W)");
  MEDNEXT_CHECK_ARG(band == kBand, "the volume engine's tile_w (plane positions per workgroup) must be 64");
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  MEDNEXT_CHECK_ARG(d < (int64_t(1) << 24) && n * c < (int64_t(1) << 40), "shape out of range");
  MEDNEXT_CHECK_ARG(d * h * w * elem_bytes(dtype) < (int64_t(1) << 31), "one (n, c) slab must be under 2 GiB");
  const int P = k / 2;
  const int acc = dtype == MEDNEXT_DTYPE_F64 ? 8 : 4;
  g->C = static_cast<int>(c);
  g->D = static_cast<int>(d);
  g->H = static_cast<int>(h);
  g->W = static_cast<int>(w);
  g->TD = static_cast<int>(std::min<int64_t>(depth_chunk, d));
  g->TDk = std::max(g->TD, k - 1);
  g->nDc = static_cast<int>(cdiv(d, g->TD));
  g->nbands = static_cast<int>(cdiv(h * w, kBand));
  g->sg = make_stage(d, h, w, static_cast<int>(band_rows(h, w)) + 2 * P, g->TDk + 2 * P, P);
  g->slabs = n * c;
  *lds = band_lds_bytes(*g, k, acc, wgrad);
  MEDNEXT_CHECK_ARG(*lds <= 64 * 1024, "depth_chunk too long: the staged planes exceed 64 KiB of LDS");
  const int64_t blocks = g->slabs * g->nbands * g->nDc;
  MEDNEXT_CHECK_ARG(blocks < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

dim3 band_grid(const BandGeom& g) { return dim3(static_cast<unsigned>(g.slabs * g.nbands * g.nDc)); }

template <typename T, int K, bool FLIP>
int launch_band_stencil(const void* x, const void* wt, const void* bias, void* y, const BandGeom& g, size_t lds,
                        hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  auto px = static_cast<const T*>(x);
  auto pw = static_cast<const T*>(wt);
  auto pb = static_cast<const T*>(bias);
  auto py = static_cast<T*>(y);
  if (bias != nullptr)
    hipLaunchKernelGGL((dw_band_stencil_kernel<T, Acc, K, FLIP, true>), band_grid(g), dim3(kBand * K), lds, st, px,
                       pw, pb, py, g);
  else
    hipLaunchKernelGGL((dw_band_stencil_kernel<T, Acc, K, FLIP, false>), band_grid(g), dim3(kBand * K), lds, st, px,
                       pw, pb, py, g);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T, bool FLIP>
int band_stencil_t(const void* x, const void* wt, const void* bias, void* y, const BandGeom& g, int k, size_t lds,
                   hipStream_t st) {
  switch (k) {
    case 1: return launch_band_stencil<T, 1, FLIP>(x, wt, bias, y, g, lds, st);
    case 3: return launch_band_stencil<T, 3, FLIP>(x, wt, bias, y, g, lds, st);
    default: return launch_band_stencil<T, 5, FLIP>(x, wt, bias, y, g, lds, st);
  }
}

template <typename T, int K>
int launch_band_wgrad(const void* x, const void* dy, void* partial, const BandGeom& g, int splits, size_t lds,
                      hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  hipLaunchKernelGGL((dw_band_wgrad_kernel<T, Acc, K>), band_grid(g), dim3(kBand * K), lds, st,
                     static_cast<const T*>(x), static_cast<const T*>(dy), static_cast<Acc*>(partial), g, splits);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T>
int band_wgrad_t(const void* x, const void* dy, void* partial, const BandGeom& g, int k, int splits, size_t lds,
                 hipStream_t st) {
  switch (k) {
    case 1: return launch_band_wgrad<T, 1>(x, dy, partial, g, splits, lds, st);
    case 3: return launch_band_wgrad<T, 3>(x, dy, partial, g, splits, lds, st);
    default: return launch_band_wgrad<T, 5>(x, dy, partial, g, splits, lds, st);
  }
}

// Stride 2. LDS a D-run of td small planes needs (gather: staged big rows +
// per-kernel-row sums; reduce: staged big rows + the band's small values, or
// the reduction buffer it is reused for).
constexpr size_t kS2GatherLds = 36 * 1024;  // preferred gather footprint (four workgroups per CU)
constexpr int kS2ReduceWorkgroups = 2048;   // reduce grid the bands-per-workgroup choice aims at

int s2band_geom(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k,
                int dtype, int td, int bpw, S2BandGeom* g) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && db >= 1 && hb >= 1 && wb >= 1 && ds >= 1 && hs >= 1 && ws >= 1,
                    "shape must be positive");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  // Small column ws reads big columns 2 ws - P .. 2 ws + P, which must stay
  // inside the staged row [-P, Wb + P).
  MEDNEXT_CHECK_ARG(2 * ws <= wb + 1, "small width must not exceed ceil(big width / 2)");
  const int64_t eb = elem_bytes(dtype);
  MEDNEXT_CHECK_ARG(db * hb * wb * eb < (int64_t(1) << 31) && ds * hs * ws * eb < (int64_t(1) << 31),
                    "one (n, c) slab must be under 2 GiB");
  MEDNEXT_CHECK_ARG(n * c < (int64_t(1) << 40) && ds < (int64_t(1) << 24), "shape out of range");
  const int P = k / 2;
  g->C = static_cast<int>(c);
  g->Db = static_cast<int>(db);
  g->Hb = static_cast<int>(hb);
  g->Wb = static_cast<int>(wb);
  g->Ds = static_cast<int>(ds);
  g->Hs = static_cast<int>(hs);
  g->Ws = static_cast<int>(ws);
  g->TD = static_cast<int>(std::min<int64_t>(td, ds));
  g->TDk = std::max(g->TD, P);
  g->nDc = static_cast<int>(cdiv(ds, g->TD));
  g->nbands = static_cast<int>(cdiv(hs * ws, kBand));
  g->bpw = std::max(1, std::min(bpw, g->nbands));
  g->nbw = static_cast<int>(cdiv(g->nbands, g->bpw));
  const int rows = static_cast<int>(2 * (band_rows(hs, ws) - 1) + k);
  g->sg = make_stage(db, hb, wb, rows, 2 * g->TDk + k - 2, P);
  g->slabs = n * c;
  return MEDNEXT_STATUS_OK;
}

size_t s2band_lds_bytes(const S2BandGeom& g, int k, int acc_bytes, bool wgrad) {
  const size_t staged = staged_elems(g.sg, k / 2);
  if (!wgrad) return (staged + static_cast<size_t>(k) * g.TDk * kBand) * acc_bytes;
  return std::max(staged + static_cast<size_t>(g.TDk) * kBand, red_elems(k, acc_bytes)) * acc_bytes;
}

// The stride-2 band plan: the longest D-run (8, 4, 2 or 1 small planes) whose
// LDS fits (the gather prefers kS2GatherLds), and for the reduce the bands per
// workgroup that bring the grid near kS2ReduceWorkgroups.
int s2band_plan(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k,
                int dtype, bool wgrad, S2BandGeom* g, size_t* lds) {
  const int acc = dtype == MEDNEXT_DTYPE_F64 ? 8 : 4;
  const size_t limit = 64 * 1024;
  int chosen = 0;
  for (int pass = 0; pass < 2 && chosen == 0; ++pass) {
    const size_t want = (!wgrad && pass == 0) ? kS2GatherLds : limit;
    for (int td : {8, 4, 2, 1}) {
      if (int st = s2band_geom(n, c, db, hb, wb, ds, hs, ws, k, dtype, td, 1, g)) return st;
      if (s2band_lds_bytes(*g, k, acc, wgrad) <= want) {
        chosen = td;
        break;
      }
    }
  }
  MEDNEXT_CHECK_ARG(chosen > 0, "stride-2 band: the staged rows exceed 64 KiB of LDS");
  int bpw = 1;
  if (wgrad) {
    S2BandGeom probe{};
    s2band_geom(n, c, db, hb, wb, ds, hs, ws, k, dtype, chosen, 1, &probe);
    const int64_t units = probe.slabs * probe.nbands * probe.nDc;
    bpw = static_cast<int>(std::max<int64_t>(1, units / kS2ReduceWorkgroups));
  }
  if (int st = s2band_geom(n, c, db, hb, wb, ds, hs, ws, k, dtype, chosen, bpw, g)) return st;
  *lds = s2band_lds_bytes(*g, k, acc, wgrad);
  const int64_t blocks = g->slabs * (wgrad ? g->nbw : g->nbands) * g->nDc;
  MEDNEXT_CHECK_ARG(blocks < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

template <typename T, int K>
int launch_s2band_gather(const void* big, const void* wt, const void* bias, void* small, const S2BandGeom& g,
                         size_t lds, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(g.slabs * g.nbands * g.nDc));
  auto pb = static_cast<const T*>(big);
  auto pw = static_cast<const T*>(wt);
  auto pbias = static_cast<const T*>(bias);
  auto ps = static_cast<T*>(small);
  if (bias != nullptr)
    hipLaunchKernelGGL((dw_s2band_gather_kernel<T, Acc, K, true>), grid, dim3(kBand * K), lds, st, pb, pw, pbias, ps,
                       g);
  else
    hipLaunchKernelGGL((dw_s2band_gather_kernel<T, Acc, K, false>), grid, dim3(kBand * K), lds, st, pb, pw, pbias,
                       ps, g);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T, int K>
int launch_s2band_wgrad(const void* big, const void* small, void* partial, const S2BandGeom& g, int splits,
                        size_t lds, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(g.slabs * g.nbw * g.nDc));
  hipLaunchKernelGGL((dw_s2band_wgrad_kernel<T, Acc, K>), grid, dim3(kBand * K), lds, st,
                     static_cast<const T*>(big), static_cast<const T*>(small), static_cast<Acc*>(partial), g, splits);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

}  // namespace

bool dw_volume_supported(int64_t h, int64_t w) { return h >= 1 && w >= 1 && h * w <= 4 * kBand; }

int dw_volume_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n, int64_t c, int64_t d,
                      int64_t h, int64_t w, int k, int dtype, bool flip, int band, int depth_chunk, hipStream_t st) {
  BandGeom g{};
  size_t lds = 0;
  if (int status = band_plan(n, c, d, h, w, k, dtype, band, depth_chunk, false, &g, &lds)) return status;
#define MEDNEXT_BAND_STENCIL(T) \
  return flip ? band_stencil_t<T, true>(x, weight, bias, y, g, k, lds, st) \
              : band_stencil_t<T, false>(x, weight, bias, y, g, k, lds, st)
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_BAND_STENCIL(float);
    case MEDNEXT_DTYPE_F64: MEDNEXT_BAND_STENCIL(double);
    case MEDNEXT_DTYPE_F16: MEDNEXT_BAND_STENCIL(f16_t);
    default: MEDNEXT_BAND_STENCIL(bf16_t);
  }
#undef MEDNEXT_BAND_STENCIL
}

int dw_volume_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int band,
                           int depth_chunk) {
  BandGeom g{};
  size_t lds = 0;
  if (band_plan(n, c, d, h, w, k, dtype, band, depth_chunk, true, &g, &lds) != MEDNEXT_STATUS_OK) return 0;
  const int64_t splits = n * g.nbands * g.nDc;
  return splits < (int64_t(1) << 31) ? static_cast<int>(splits) : 0;
}

int dw_volume_wgrad(const void* x, const void* dy, void* partial, int64_t n, int64_t c, int64_t d, int64_t h,
                    int64_t w, int k, int dtype, int band, int depth_chunk, hipStream_t st) {
  BandGeom g{};
  size_t lds = 0;
  if (int status = band_plan(n, c, d, h, w, k, dtype, band, depth_chunk, true, &g, &lds)) return status;
  const int64_t splits = n * g.nbands * g.nDc;
  MEDNEXT_CHECK_ARG(splits < (int64_t(1) << 31), "too many partials");
  const int s = static_cast<int>(splits);
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: return band_wgrad_t<float>(x, dy, partial, g, k, s, lds, st);
    case MEDNEXT_DTYPE_F64: return band_wgrad_t<double>(x, dy, partial, g, k, s, lds, st);
    case MEDNEXT_DTYPE_F16: return band_wgrad_t<f16_t>(x, dy, partial, g, k, s, lds, st);
    default: return band_wgrad_t<bf16_t>(x, dy, partial, g, k, s, lds, st);
  }
}

bool dw_s2band_chosen(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                      int64_t ws, int k, int dtype) {
  // Measured on MI355X (bf16, MedNeXt down / up shapes): the band kernels win
  // for k = 5 and for k = 3 up to 64 columns when the big rows load in
  // 4-column chunks; the row-task kernels win for k = 3 at 128 columns and for
  // odd widths (the up blocks' 2s - 1), whose staging goes element by element.
  const bool preferred = wb % 4 == 0 && (k == 5 || (k == 3 && wb <= 64));
  return preferred && dw_s2band_supported(n, c, db, hb, wb, ds, hs, ws, k, dtype);
}

bool dw_s2band_supported(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                         int64_t ws, int k, int dtype) {
  S2BandGeom g{};
  size_t lds = 0;
  return s2band_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, false, &g, &lds) == MEDNEXT_STATUS_OK &&
         s2band_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, true, &g, &lds) == MEDNEXT_STATUS_OK &&
         n * g.nbw * g.nDc < (int64_t(1) << 31);
}

int dw_s2band_gather(const void* big, const void* weight, const void* bias, void* small, int64_t n, int64_t c,
                     int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, int dtype,
                     hipStream_t st) {
  S2BandGeom g{};
  size_t lds = 0;
  if (int status = s2band_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, false, &g, &lds)) return status;
#define MEDNEXT_S2BAND_GATHER(T)                                                   \
  switch (k) {                                                                     \
    case 1: return launch_s2band_gather<T, 1>(big, weight, bias, small, g, lds, st); \
    case 3: return launch_s2band_gather<T, 3>(big, weight, bias, small, g, lds, st); \
    default: return launch_s2band_gather<T, 5>(big, weight, bias, small, g, lds, st); \
  }
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_S2BAND_GATHER(float)
    case MEDNEXT_DTYPE_F64: MEDNEXT_S2BAND_GATHER(double)
    case MEDNEXT_DTYPE_F16: MEDNEXT_S2BAND_GATHER(f16_t)
    default: MEDNEXT_S2BAND_GATHER(bf16_t)
  }
#undef MEDNEXT_S2BAND_GATHER
}

int dw_s2band_wgrad_splits(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                           int64_t ws, int k, int dtype) {
  S2BandGeom g{};
  size_t lds = 0;
  if (s2band_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, true, &g, &lds) != MEDNEXT_STATUS_OK) return 0;
  const int64_t splits = n * g.nbw * g.nDc;
  return splits < (int64_t(1) << 31) ? static_cast<int>(splits) : 0;
}

int dw_s2band_wgrad(const void* big, const void* small, void* partial, int64_t n, int64_t c, int64_t db, int64_t hb,
                    int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, int dtype, hipStream_t st) {
  S2BandGeom g{};
  size_t lds = 0;
  if (int status = s2band_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, true, &g, &lds)) return status;
  const int64_t splits = n * g.nbw * g.nDc;
  MEDNEXT_CHECK_ARG(splits < (int64_t(1) << 31), "too many partials");
  const int s = static_cast<int>(splits);
#define MEDNEXT_S2BAND_WGRAD(T)                                                  \
  switch (k) {                                                                   \
    case 1: return launch_s2band_wgrad<T, 1>(big, small, partial, g, s, lds, st); \
    case 3: return launch_s2band_wgrad<T, 3>(big, small, partial, g, s, lds, st); \
    default: return launch_s2band_wgrad<T, 5>(big, small, partial, g, s, lds, st); \
  }
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_S2BAND_WGRAD(float)
    case MEDNEXT_DTYPE_F64: MEDNEXT_S2BAND_WGRAD(double)
    case MEDNEXT_DTYPE_F16: MEDNEXT_S2BAND_WGRAD(f16_t)
    default: MEDNEXT_S2BAND_WGRAD(bf16_t)
  }
#undef MEDNEXT_S2BAND_WGRAD
}

}  // namespace mednext
