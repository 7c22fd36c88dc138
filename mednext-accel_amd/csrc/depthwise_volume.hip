// Depthwise Conv3d (stride 1, odd cubic kernel, zero "same" padding) on small
// planes: H * W <= 256 elements, the MedNeXt stages at 16^3 and 8^3. Every
// dtype; fp32 accumulation (fp64 for fp64).
//
// At these sizes the tiled kernels leave most lanes idle (a 16 x 16 plane is
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
//     splits (one per (n, band, D-run)).
// The first and last k - 1 planes of the walk are unrolled with only the taps
// whose output (forward) or grad_output (weight gradient) plane exists in the
// D-run, so no FMA is spent on the zero padding along D.
#include "cdna4.h"
#include "common.h"
#include "depthwise_volume.h"

#include <algorithm>

namespace mednext {
namespace {

constexpr int kBand = 64;  // plane positions per workgroup: one wave's lanes
constexpr int kFillBatch = 8;  // loads in flight per thread while staging

struct BandGeom {
  int C, D, H, W;
  int TD;        // output planes per D-run
  int TDk;       // planes the lanes walk: max(TD, k - 1); planes past the D-run are zero / not stored
  int nDc;       // D-runs per slab
  int nbands;    // bands per plane
  int SR;        // staged rows per band: the most rows a band spans + 2P
  uint32_t wp_magic;     // ceil(2^31 / (W + 2P))
  uint32_t plane_magic;  // ceil(2^31 / (SR * (W + 2P)))
  uint32_t w4_magic;     // ceil(2^31 / (W / 4)) (W % 4 == 0 only)
  uint32_t sr_magic;     // ceil(2^31 / SR)
  int64_t slabs;
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

// Stage rows [hb0 - P, hb0 - P + SR) x columns [-P, W + P) of the planes
// [d0 - P, d0 + TDk + P) of one slab into lds[pd][row][col], zero outside the
// tensor. Consecutive threads take consecutive columns of a row. Loads go
// through a raw buffer resource over the slab, out-of-tensor elements read the
// out-of-range offset (zero), so each thread issues kFillBatch loads back to
// back with no branches before its first store.
template <typename T, typename Acc, int P>
__device__ inline void fill_band(Acc* __restrict__ lds, const T* __restrict__ x, const BandGeom& g, int64_t slab,
                                 int d0, int hb0, int nthreads) {
  const int Wp = g.W + 2 * P;
  const int per_plane = g.SR * Wp;
  const int total = (g.TDk + 2 * P) * per_plane;
  const int plane = g.H * g.W;
  const __amdgpu_buffer_rsrc_t src =
      slab_rsrc(x + slab * g.D * plane, static_cast<uint32_t>(g.D * plane * static_cast<int>(sizeof(T))));
  for (int base = 0; base < total; base += nthreads * kFillBatch) {
    Acc v[kFillBatch];
#pragma unroll
    for (int b = 0; b < kFillBatch; ++b) {
      v[b] = Acc(0);
      if (base + b * nthreads >= total) break;  // uniform: no load for slots past the staged block
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      const int pd = div_magic(e, g.plane_magic);
      const int r = e - pd * per_plane;
      const int sr = div_magic(r, g.wp_magic);
      const int gw = r - sr * Wp - P;
      const int gh = hb0 + sr - P;
      const int gd = d0 + pd - P;
      const bool ok = e < total && gd >= 0 && gd < g.D && gh >= 0 && gh < g.H && gw >= 0 && gw < g.W;
      v[b] = BufIo<T>::ld(src, boff<T>(ok, gd * plane + gh * g.W + gw));
    }
#pragma unroll
    for (int b = 0; b < kFillBatch; ++b) {
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      if (e < total) lds[e] = v[b];
    }
  }
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

// fill_band for W % 4 == 0: the interior of each staged row is loaded in
// 4-column chunks (a quarter of the load instructions and index arithmetic),
// and the 2P padding columns of every row are written as zeros.
constexpr int kChunkBatch = 4;

template <typename T, typename Acc, int P>
__device__ inline void fill_band_w4(Acc* __restrict__ lds, const T* __restrict__ x, const BandGeom& g, int64_t slab,
                                    int d0, int hb0, int nthreads) {
  const int Wp = g.W + 2 * P, W4 = g.W >> 2;
  const int rows = (g.TDk + 2 * P) * g.SR;
  const int total = rows * W4;
  const int plane = g.H * g.W;
  const __amdgpu_buffer_rsrc_t src =
      slab_rsrc(x + slab * g.D * plane, static_cast<uint32_t>(g.D * plane * static_cast<int>(sizeof(T))));
  for (int base = 0; base < total; base += nthreads * kChunkBatch) {
    Acc v[kChunkBatch][4];
    int dst[kChunkBatch];  // LDS element offset of the chunk, -1: nothing to store
#pragma unroll
    for (int b = 0; b < kChunkBatch; ++b) dst[b] = -1;
#pragma unroll
    for (int b = 0; b < kChunkBatch; ++b) {
      if (base + b * nthreads >= total) break;  // uniform
      const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
      const int row = div_magic(e, g.w4_magic);
      const int cx = e - row * W4;
      const int pd = div_magic(row, g.sr_magic);
      const int sr = row - pd * g.SR;
      const int gh = hb0 + sr - P;
      const int gd = d0 + pd - P;
      const bool ok = e < total && gd >= 0 && gd < g.D && gh >= 0 && gh < g.H;
      BufIo4<T>::ld(src, boff<T>(ok, gd * plane + gh * g.W + 4 * cx), v[b]);
      dst[b] = e < total ? row * Wp + P + 4 * cx : -1;
    }
#pragma unroll
    for (int b = 0; b < kChunkBatch; ++b) {
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
        lds[row * Wp + P + g.W + j] = Acc(0);
      }
    }
  }
}

template <typename T, typename Acc, int P>
__device__ inline void stage_input(Acc* __restrict__ lds, const T* __restrict__ x, const BandGeom& g, int64_t slab,
                                   int d0, int hb0, int nthreads) {
  if ((g.W & 3) == 0)
    fill_band_w4<T, Acc, P>(lds, x, g, slab, d0, hb0, nthreads);
  else
    fill_band<T, Acc, P>(lds, x, g, slab, d0, hb0, nthreads);
}

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

// The weight gradient's staging: grad_output of the band into ds[od][l]
// (CW consecutive positions per load) around the input planes' staging.
constexpr int kDyBatch = 4;

template <typename T, typename Acc, int CW>
__device__ inline void dy_batch_load(Acc (&v)[kDyBatch][CW], __amdgpu_buffer_rsrc_t src, const BandGeom& g,
                                     const BandTile& t, int base, int nthreads) {
  const int hw = g.H * g.W;
  const int nb = min(kBand, hw - t.p0);
  constexpr int per_plane = kBand / CW;
  const int total = g.TDk * per_plane;
#pragma unroll
  for (int b = 0; b < kDyBatch; ++b) {
    const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
    const int od = e / per_plane, l = (e % per_plane) * CW;
    const uint32_t off = boff<T>(e < total && od < t.nd && l < nb, (t.d0 + od) * hw + t.p0 + l);
    if constexpr (CW == 4) {
      BufIo4<T>::ld(src, off, v[b]);
    } else {
      v[b][0] = BufIo<T>::ld(src, off);
    }
  }
}

template <typename Acc, int CW>
__device__ inline void dy_batch_store(Acc* __restrict__ ds, const Acc (&v)[kDyBatch][CW], const BandGeom& g,
                                      int base, int nthreads) {
  constexpr int per_plane = kBand / CW;
  const int total = g.TDk * per_plane;
#pragma unroll
  for (int b = 0; b < kDyBatch; ++b) {
    const int e = base + b * nthreads + static_cast<int>(threadIdx.x);
    if (e < total) {
#pragma unroll
      for (int j = 0; j < CW; ++j) ds[(e / per_plane) * kBand + (e % per_plane) * CW + j] = v[b][j];
    }
  }
}

template <typename T, typename Acc, int P, int CW>
__device__ inline void stage_band_dy(Acc* __restrict__ xs, Acc* __restrict__ ds, const T* __restrict__ x,
                                     const T* __restrict__ dy, const BandGeom& g, const BandTile& t, int nthreads) {
  const int hw = g.H * g.W;
  const __amdgpu_buffer_rsrc_t src =
      slab_rsrc(dy + t.slab * g.D * hw, static_cast<uint32_t>(g.D * hw * static_cast<int>(sizeof(T))));
  const int total = g.TDk * (kBand / CW);
  Acc v[kDyBatch][CW];
  dy_batch_load<T, Acc, CW>(v, src, g, t, 0, nthreads);
  stage_input<T, Acc, P>(xs, x, g, t.slab, t.d0, t.hb0, nthreads);
  dy_batch_store<Acc, CW>(ds, v, g, 0, nthreads);
  for (int base = nthreads * kDyBatch; base < total; base += nthreads * kDyBatch) {
    dy_batch_load<T, Acc, CW>(v, src, g, t, base, nthreads);
    dy_batch_store<Acc, CW>(ds, v, g, base, nthreads);
  }
}

template <typename Acc, int K>
__device__ inline void load_row(Acc (&xv)[K], const Acc* __restrict__ p) {
#pragma unroll
  for (int kw = 0; kw < K; ++kw) xv[kw] = p[kw];
}

template <typename Acc, int K>
__device__ inline void shift_ring(Acc (&ring)[K]) {
#pragma unroll
  for (int j = K - 1; j > 0; --j) ring[j] = ring[j - 1];
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
  const int per_plane = g.SR * Wp;
  Acc* const rows = xs + (g.TDk + 2 * P) * per_plane;  // [K][TDk][kBand] per-kernel-row sums

  const BandTile t = band_tile(g);
  stage_input<T, Acc, P>(xs, x, g, t.slab, t.d0, t.hb0, NT);

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
  const int hw = g.H * g.W;
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

// Values per lane (one kernel row's taps + the bias sum) reduced per LDS
// round: all of them, except fp64 at k = 5, whose 26 values per lane are
// reduced in two rounds to stay within the staged LDS footprint.
template <typename Acc, int K>
constexpr int band_red_values() {
  return sizeof(Acc) == 8 && K == 5 ? 13 : K * K + 1;
}

template <typename T, typename Acc, int K>
__global__ __launch_bounds__(kBand * K) void dw_band_wgrad_kernel(const T* __restrict__ x,
                                                                  const T* __restrict__ dy,
                                                                  Acc* __restrict__ partial, BandGeom g,
                                                                  int splits) {
  constexpr int P = K / 2, K2 = K * K, K3 = K2 * K, NT = kBand * K;
  constexpr int NACC = K2 + 1;  // this kernel row's taps + the bias sum
  constexpr int RT = band_red_values<Acc, K>();
  constexpr int PITCH = RT | 1;  // odd: lane-strided LDS accesses hit distinct banks
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Wp = g.W + 2 * P;
  const int per_plane = g.SR * Wp;
  Acc* const ds = xs + (g.TDk + 2 * P) * per_plane;  // [TDk][kBand] grad_output of the band

  const BandTile t = band_tile(g);
  const int hw = g.H * g.W;
  // grad_output of the band, ds[od][l] for the band's position l: the first
  // batch of loads is issued before the input planes are staged and stays in
  // flight meanwhile. With W % 4 == 0 a band is whole 4-position chunks.
  if ((g.W & 3) == 0)
    stage_band_dy<T, Acc, P, 4>(xs, ds, x, dy, g, t, NT);
  else
    stage_band_dy<T, Acc, P, 1>(xs, ds, x, dy, g, t, NT);
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

  // Per-wave fixed-order reduction over the 64 lanes, through LDS that aliases
  // the staged planes: value r0 + i of lane l at red[l * PITCH + i].
  Acc* __restrict__ red = xs + kh * kBand * PITCH;
  const int64_t c = t.slab % g.C, n = t.slab / g.C;
  const int64_t split = (n * g.nbands + t.band) * g.nDc + t.dc;
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

int64_t band_rows(int64_t h, int64_t w) {
  const int64_t hw = h * w;
  int64_t most = 1;
  for (int64_t p0 = 0; p0 < hw; p0 += kBand) {
    const int64_t last = std::min<int64_t>(p0 + kBand, hw) - 1;
    most = std::max<int64_t>(most, last / w - p0 / w + 1);
  }
  return most;
}

size_t band_lds_bytes(const BandGeom& g, int k, int acc_bytes, bool wgrad) {
  const int P = k / 2;
  const size_t staged = static_cast<size_t>(g.TDk + 2 * P) * g.SR * (g.W + 2 * P);
  if (!wgrad) return (staged + static_cast<size_t>(k) * g.TDk * kBand) * acc_bytes;
  const int rt = acc_bytes == 8 && k == 5 ? 13 : k * k + 1;
  const size_t red = static_cast<size_t>(k) * kBand * (rt | 1);
  return std::max(staged + static_cast<size_t>(g.TDk) * kBand, red) * acc_bytes;
}

uint32_t magic31(int64_t d) { return static_cast<uint32_t>(((int64_t(1) << 31) + d - 1) / d); }

int band_plan(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int band, int depth_chunk,
              bool wgrad, BandGeom* g, size_t* lds) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h >= 1 && w >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  MEDNEXT_CHECK_ARG(h * w <= 4 * kBand, "the volume engine takes planes of at most 256 elements (H * W)");
  MEDNEXT_CHECK_ARG(band == kBand, "the volume engine's tile_w (plane positions per workgroup) must be 64");
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  MEDNEXT_CHECK_ARG(d < (int64_t(1) << 24) && n * c < (int64_t(1) << 40), "shape out of range");
  const int64_t elem = dtype == MEDNEXT_DTYPE_F64 ? 8 : dtype == MEDNEXT_DTYPE_F32 ? 4 : 2;
  MEDNEXT_CHECK_ARG(d * h * w * elem < (int64_t(1) << 31), "one (n, c) slab must be under 2 GiB");
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
  g->SR = static_cast<int>(band_rows(h, w)) + 2 * P;
  g->wp_magic = magic31(w + 2 * P);
  g->plane_magic = magic31(static_cast<int64_t>(g->SR) * (w + 2 * P));
  g->w4_magic = magic31(std::max<int64_t>(1, w / 4));
  g->sr_magic = magic31(g->SR);
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

}  // namespace mednext
