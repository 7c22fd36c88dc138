// Depthwise Conv3d (stride 1, odd cubic kernel, zero "same" padding) for gfx950:
// forward, input gradient (same stencil with flipped taps) and weight gradient
// with the bias gradient fused in the same pass.
//
// Work decomposition (all three kernels): one workgroup owns one (n, c) slab, a
// run of `depth_chunk` output planes and one TH x TW tile of each plane. Input
// planes stream along D through an LDS halo tile of (TH + 2p) x (TW + 8)
// elements (converted to the accumulation type on the way in). Each thread
// owns a kRH x 4 patch of outputs. Along D the forward/dgrad kernels scatter:
// every input plane is read from LDS once and added into k rotating
// per-output-plane register accumulators, so an output plane is complete (and
// written) k-1 input planes after its first contribution. The weight-gradient
// kernel keeps a k-plane ring of grad_output values in registers instead and
// accumulates k^3 tap sums per thread, reduced per workgroup into a fp32/fp64
// partial and then summed over workgroups in a fixed order (deterministic).
#include "cdna4.h"
#include "common.h"
#include "depthwise_mfma.h"
#include "depthwise_volume.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace mednext {
namespace {

constexpr int kMaxThreads = 256;
constexpr int kRH = 2;  // output rows per thread

struct DwGeom {
  int C, D, H, W;
  int TD;   // output planes per workgroup
  int TWt;  // threads along w; tile width TW = 4 * TWt
  int THt;  // threads along h holding outputs; tile height TH = kRH * THt
  int nDc, nHt, nWt;
};

struct TileIdx {
  int64_t nc;
  int c, n, d0, th0, tw0, dc, ht, wt;
};

__device__ inline TileIdx tile_of_block(const DwGeom& g) {
  TileIdx t;
  int64_t bid = blockIdx.x;
  t.wt = static_cast<int>(bid % g.nWt);
  bid /= g.nWt;
  t.ht = static_cast<int>(bid % g.nHt);
  bid /= g.nHt;
  t.dc = static_cast<int>(bid % g.nDc);
  bid /= g.nDc;
  t.nc = bid;
  t.c = static_cast<int>(bid % g.C);
  t.n = static_cast<int>(bid / g.C);
  t.d0 = t.dc * g.TD;
  t.th0 = t.ht * kRH * g.THt;
  t.tw0 = t.wt * 4 * g.TWt;
  return t;
}

// 16-byte LDS accesses (the row stride is a multiple of 4 elements and the
// buffer is 16-byte aligned, so every group of 4 starts on a 16-byte boundary).
__device__ inline void lds_store4(float* dst, const float v[4]) {
  *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
}
__device__ inline void lds_store4(double* dst, const double v[4]) {
  reinterpret_cast<double2*>(dst)[0] = make_double2(v[0], v[1]);
  reinterpret_cast<double2*>(dst)[1] = make_double2(v[2], v[3]);
}
__device__ inline void lds_load4(const float* src, float v[4]) {
  const float4 a = *reinterpret_cast<const float4*>(src);
  v[0] = a.x;
  v[1] = a.y;
  v[2] = a.z;
  v[3] = a.w;
}
__device__ inline void lds_load4(const double* src, double v[4]) {
  const double2 a = reinterpret_cast<const double2*>(src)[0];
  const double2 b = reinterpret_cast<const double2*>(src)[1];
  v[0] = a.x;
  v[1] = a.y;
  v[2] = b.x;
  v[3] = b.y;
}

// Fill the LDS halo tile with input plane `di` (zeros outside the volume).
// LDS column j holds w = tw0 - 4 + j; LDS row r holds h = th0 - P + r.
template <typename T, typename Acc, int P, bool VEC>
__device__ inline void fill_plane(Acc* __restrict__ lds, const T* __restrict__ src, int di,
                                  const DwGeom& g, int th0, int tw0, int lrows, int rs) {
  const int nthreads = blockDim.x;
  const bool plane_ok = di >= 0 && di < g.D;
  const T* __restrict__ p = src + static_cast<int64_t>(plane_ok ? di : 0) * g.H * g.W;
  if constexpr (VEC) {
    const int groups = rs >> 2;
    const int total = lrows * groups;
    for (int e = threadIdx.x; e < total; e += nthreads) {
      const int rr = e / groups;
      const int gq = e - rr * groups;
      const int h = th0 - P + rr;
      const int w = tw0 - 4 + 4 * gq;
      Acc v[4] = {Acc(0), Acc(0), Acc(0), Acc(0)};
      // W % 4 == 0 and w % 4 == 0: a group is entirely inside or outside.
      if (plane_ok && h >= 0 && h < g.H && w >= 0 && w < g.W) {
        load4<T, Acc>(p + static_cast<int64_t>(h) * g.W + w, v);
      }
      lds_store4(lds + rr * rs + 4 * gq, v);
    }
  } else {
    const int total = lrows * rs;
    for (int e = threadIdx.x; e < total; e += nthreads) {
      const int rr = e / rs;
      const int cc = e - rr * rs;
      const int h = th0 - P + rr;
      const int w = tw0 - 4 + cc;
      Acc v = Acc(0);
      if (plane_ok && h >= 0 && h < g.H && w >= 0 && w < g.W) {
        v = Cvt<T, Acc>::load(p[static_cast<int64_t>(h) * g.W + w]);
      }
      lds[rr * rs + cc] = v;
    }
  }
}

// Read this thread's (kRH + 2P) x 12 input window from the LDS tile: columns
// 4*tx .. 4*tx+11 hold w = tw0 + 4*tx - 4 .. tw0 + 4*tx + 7.
template <typename Acc, int P>
__device__ inline void read_window(const Acc* __restrict__ lds, int ty, int tx, int rs,
                                   Acc in[kRH + 2 * P][12]) {
#pragma unroll
  for (int j = 0; j < kRH + 2 * P; ++j) {
    const Acc* row = lds + (ty * kRH + j) * rs + 4 * tx;
    lds_load4(row, &in[j][0]);
    lds_load4(row + 4, &in[j][4]);
    lds_load4(row + 8, &in[j][8]);
  }
}

// Per-channel taps, uniform across the workgroup. bf16 taps are fetched as
// 32-bit words and split with integer shifts so they stay in scalar registers
// (there is no 16-bit scalar load); the weight buffer must be 4-byte aligned.
template <typename T, typename Acc, int K3, bool FLIP>
__device__ inline void load_taps(const T* __restrict__ wt, int c, int channels, Acc wr[K3]) {
  if constexpr (std::is_same<T, bf16_t>::value) {
    const uint32_t* __restrict__ words = reinterpret_cast<const uint32_t*>(wt);
    const int64_t e0 = static_cast<int64_t>(c) * K3;
    const int64_t total = static_cast<int64_t>(channels) * K3;
#pragma unroll
    for (int i = 0; i < K3; ++i) {
      const int64_t e = e0 + (FLIP ? K3 - 1 - i : i);
      if (e + 1 == total && (e & 1) == 0) {
        // Last tap of an odd-length buffer: its 32-bit word would extend past
        // the end, so read the 16-bit element itself.
        wr[i] = bf16_to_f32(wt[e].bits);
      } else {
        const uint32_t word = words[e >> 1];
        wr[i] = __uint_as_float((e & 1) ? (word & 0xffff0000u) : (word << 16));
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < K3; ++i) {
      wr[i] = Cvt<T, Acc>::load(wt[static_cast<int64_t>(c) * K3 + (FLIP ? K3 - 1 - i : i)]);
    }
  }
}

template <typename T, typename Acc, int K, bool FLIP, bool VEC, bool BIAS>
__global__ __launch_bounds__(kMaxThreads) void dw_stencil_kernel(const T* __restrict__ x,
                                                                 const T* __restrict__ wt,
                                                                 const T* __restrict__ bias,
                                                                 T* __restrict__ y, DwGeom g) {
  constexpr int P = K / 2;
  constexpr int K3 = K * K * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* lds = reinterpret_cast<Acc*>(smem_raw);

  const TileIdx t = tile_of_block(g);
  const int rs = 4 * g.TWt + 8;
  const int lrows = kRH * g.THt + 2 * P;
  const int tx = threadIdx.x % g.TWt;
  const int ty = threadIdx.x / g.TWt;
  const bool owner = ty < g.THt;

  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const T* __restrict__ xnc = x + t.nc * g.D * plane;
  T* __restrict__ ync = y + t.nc * g.D * plane;

  Acc wr[K3];
  load_taps<T, Acc, K3, FLIP>(wt, t.c, g.C, wr);
  Acc b0 = Acc(0);
  if constexpr (BIAS) b0 = Cvt<T, Acc>::load(bias[t.c]);

  Acc acc[K][kRH][4];
#pragma unroll
  for (int s = 0; s < K; ++s)
#pragma unroll
    for (int r = 0; r < kRH; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) acc[s][r][v] = Acc(0);

  const int nplanes = g.TD + K - 1;
  for (int q = 0; q < nplanes; q += K) {
#pragma unroll
    for (int s = 0; s < K; ++s) {
      const int i = q + s;
      if (i >= nplanes) break;
      __syncthreads();
      fill_plane<T, Acc, P, VEC>(lds, xnc, t.d0 - P + i, g, t.th0, t.tw0, lrows, rs);
      __syncthreads();
      if (owner) {
        Acc in[kRH + 2 * P][12];
        read_window<Acc, P>(lds, ty, tx, rs, in);
        // Input plane i feeds output plane o = i - kd through tap kd.
#pragma unroll
        for (int kd = 0; kd < K; ++kd) {
          const int slot = ((s - kd) % K + K) % K;
#pragma unroll
          for (int kh = 0; kh < K; ++kh)
#pragma unroll
            for (int kw = 0; kw < K; ++kw) {
              const Acc wv = wr[(kd * K + kh) * K + kw];
#pragma unroll
              for (int r = 0; r < kRH; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[slot][r][v] += in[r + kh][4 - P + v + kw] * wv;
            }
        }
      }
      // Output plane o = i - (K - 1) has now received all K input planes.
      const int o = i - (K - 1);
      const int cs = (s + 1) % K;
      if (owner && o >= 0 && o < g.TD && t.d0 + o < g.D) {
        T* __restrict__ dst = ync + static_cast<int64_t>(t.d0 + o) * plane;
#pragma unroll
        for (int r = 0; r < kRH; ++r) {
          const int h = t.th0 + ty * kRH + r;
          const int w = t.tw0 + 4 * tx;
          if (h >= g.H) continue;
          Acc out[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) out[v] = acc[cs][r][v] + b0;
          T* rowp = dst + static_cast<int64_t>(h) * g.W + w;
          if constexpr (VEC) {
            if (w < g.W) store4<T, Acc>(rowp, out);
          } else {
#pragma unroll
            for (int v = 0; v < 4; ++v)
              if (w + v < g.W) rowp[v] = Cvt<T, Acc>::store(out[v]);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < kRH; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[cs][r][v] = Acc(0);
    }
  }
}

template <typename T, typename Acc, int K, bool VEC>
__global__ __launch_bounds__(kMaxThreads) void dw_wgrad_kernel(const T* __restrict__ x,
                                                               const T* __restrict__ dy,
                                                               Acc* __restrict__ partial,
                                                               DwGeom g, int splits) {
  constexpr int P = K / 2;
  constexpr int K3 = K * K * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* lds = reinterpret_cast<Acc*>(smem_raw);
  __shared__ Acc red[kMaxThreads / 64][K3 + 1];

  const TileIdx t = tile_of_block(g);
  const int rs = 4 * g.TWt + 8;
  const int lrows = kRH * g.THt + 2 * P;
  const int tx = threadIdx.x % g.TWt;
  const int ty = threadIdx.x / g.TWt;
  const bool owner = ty < g.THt;

  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const T* __restrict__ xnc = x + t.nc * g.D * plane;
  const T* __restrict__ dync = dy + t.nc * g.D * plane;

  Acc acc[K3 + 1];
#pragma unroll
  for (int i = 0; i < K3 + 1; ++i) acc[i] = Acc(0);
  Acc dyr[K][kRH][4];
#pragma unroll
  for (int s = 0; s < K; ++s)
#pragma unroll
    for (int r = 0; r < kRH; ++r)
#pragma unroll
      for (int v = 0; v < 4; ++v) dyr[s][r][v] = Acc(0);

  const int h_base = t.th0 + ty * kRH;
  const int w_base = t.tw0 + 4 * tx;
  const int nplanes = g.TD + K - 1;
  for (int q = 0; q < nplanes; q += K) {
#pragma unroll
    for (int s = 0; s < K; ++s) {
      const int i = q + s;
      if (i >= nplanes) break;
      // grad_output plane o = i enters the ring at slot i % K == s.
      {
        const bool plane_ok = owner && i < g.TD && t.d0 + i < g.D;
        const T* __restrict__ src = dync + static_cast<int64_t>(plane_ok ? t.d0 + i : 0) * plane;
#pragma unroll
        for (int r = 0; r < kRH; ++r) {
          const int h = h_base + r;
          Acc v4[4] = {Acc(0), Acc(0), Acc(0), Acc(0)};
          if (plane_ok && h < g.H) {
            const T* rowp = src + static_cast<int64_t>(h) * g.W + w_base;
            if constexpr (VEC) {
              if (w_base < g.W) load4<T, Acc>(rowp, v4);
            } else {
#pragma unroll
              for (int v = 0; v < 4; ++v)
                if (w_base + v < g.W) v4[v] = Cvt<T, Acc>::load(rowp[v]);
            }
          }
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            dyr[s][r][v] = v4[v];
            acc[K3] += v4[v];
          }
        }
      }
      __syncthreads();
      fill_plane<T, Acc, P, VEC>(lds, xnc, t.d0 - P + i, g, t.th0, t.tw0, lrows, rs);
      __syncthreads();
      if (owner) {
        Acc in[kRH + 2 * P][12];
        read_window<Acc, P>(lds, ty, tx, rs, in);
        // Input plane i pairs with grad_output plane o = i - kd through tap kd.
#pragma unroll
        for (int kd = 0; kd < K; ++kd) {
          const int slot = ((s - kd) % K + K) % K;
#pragma unroll
          for (int kh = 0; kh < K; ++kh)
#pragma unroll
            for (int kw = 0; kw < K; ++kw) {
              Acc sum = acc[(kd * K + kh) * K + kw];
#pragma unroll
              for (int r = 0; r < kRH; ++r)
#pragma unroll
                for (int v = 0; v < 4; ++v) sum += in[r + kh][4 - P + v + kw] * dyr[slot][r][v];
              acc[(kd * K + kh) * K + kw] = sum;
            }
        }
      }
    }
  }

  // Workgroup reduction: fixed butterfly inside each wave, then waves in order.
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
#pragma unroll
  for (int i = 0; i < K3 + 1; ++i) {
    const Acc v = wave_sum(acc[i]);
    if (lane == 0) red[wave][i] = v;
  }
  __syncthreads();
  const int64_t split = ((static_cast<int64_t>(t.n) * g.nDc + t.dc) * g.nHt + t.ht) * g.nWt + t.wt;
  for (int i = threadIdx.x; i < K3 + 1; i += blockDim.x) {
    Acc v = red[0][i];
    for (int wv = 1; wv < nwaves; ++wv) v += red[wv][i];
    partial[(static_cast<int64_t>(t.c) * (K3 + 1) + i) * splits + split] = v;
  }
}

// Sum the per-workgroup partials of one (channel, tap) in a fixed order: one
// wave per tap, lane j takes partials j, j + 64, ... in fp64, then a fixed
// butterfly. Partials are laid out [C][k^3 + 1][splits]; tap k^3 is the bias.
template <typename T, typename Acc>
__global__ __launch_bounds__(256) void dw_wgrad_finish_kernel(const Acc* __restrict__ partial,
                                                              T* __restrict__ dw,
                                                              T* __restrict__ db, int channels,
                                                              int splits, int k3) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (item >= static_cast<int64_t>(channels) * (k3 + 1)) return;
  const Acc* p = partial + item * splits;
  double s = 0.0;
  for (int j = lane; j < splits; j += 64) s += static_cast<double>(p[j]);
  s = wave_sum(s);
  if (lane == 0) {
    const int64_t c = item / (k3 + 1);
    const int t = static_cast<int>(item - c * (k3 + 1));
    if (t < k3) {
      dw[c * k3 + t] = Cvt<T, Acc>::store(static_cast<Acc>(s));
    } else if (db != nullptr) {
      db[c] = Cvt<T, Acc>::store(static_cast<Acc>(s));
    }
  }
}

// The same sums for few partials per tap: one thread per (channel, tap), the
// partials added in index order in fp64.
template <typename T, typename Acc>
__global__ __launch_bounds__(256) void dw_wgrad_finish_few_kernel(const Acc* __restrict__ partial,
                                                                  T* __restrict__ dw, T* __restrict__ db,
                                                                  int channels, int splits, int k3) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (item >= static_cast<int64_t>(channels) * (k3 + 1)) return;
  const Acc* p = partial + item * splits;
  double s = 0.0;
  for (int j = 0; j < splits; ++j) s += static_cast<double>(p[j]);
  const int64_t c = item / (k3 + 1);
  const int t = static_cast<int>(item - c * (k3 + 1));
  if (t < k3) {
    dw[c * k3 + t] = Cvt<T, Acc>::store(static_cast<Acc>(s));
  } else if (db != nullptr) {
    db[c] = Cvt<T, Acc>::store(static_cast<Acc>(s));
  }
}

// Partials per tap up to which one thread sums a tap (above it, a wave per tap).
constexpr int kFinishFewSplits = 16;

template <typename T, typename Acc>
int launch_finish(const Acc* part, void* dw, void* db, int64_t c, int splits, int k3,
                  hipStream_t st) {
  const int64_t items = c * (k3 + 1);
  if (splits <= kFinishFewSplits) {
    hipLaunchKernelGGL((dw_wgrad_finish_few_kernel<T, Acc>), dim3(static_cast<unsigned>(cdiv(items, 256))),
                       dim3(256), 0, st, part, static_cast<T*>(dw), static_cast<T*>(db), static_cast<int>(c),
                       splits, k3);
    MEDNEXT_CHECK_LAUNCH();
    return MEDNEXT_STATUS_OK;
  }
  hipLaunchKernelGGL((dw_wgrad_finish_kernel<T, Acc>), dim3(static_cast<unsigned>(cdiv(items, 4))),
                     dim3(256), 0, st, part, static_cast<T*>(dw), static_cast<T*>(db),
                     static_cast<int>(c), splits, k3);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

// launch_finish for a dtype known only at run time (partials in its accumulation type).
int finish_partials(int dtype, const void* part, void* dw, void* db, int64_t c, int splits, int k3, hipStream_t st) {
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: return launch_finish<float, float>(static_cast<const float*>(part), dw, db, c, splits, k3, st);
    case MEDNEXT_DTYPE_F64:
      return launch_finish<double, double>(static_cast<const double*>(part), dw, db, c, splits, k3, st);
    case MEDNEXT_DTYPE_F16: return launch_finish<f16_t, float>(static_cast<const float*>(part), dw, db, c, splits, k3, st);
    default: return launch_finish<bf16_t, float>(static_cast<const float*>(part), dw, db, c, splits, k3, st);
  }
}

// ------------------------------------------------------------------ host side

struct Plan {
  DwGeom g;
  int threads;
  size_t lds_bytes;
  int64_t blocks;
  int splits;  // workgroups per channel (wgrad partial count)
};

int make_plan(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int acc_bytes,
              int tile_w, int depth_chunk, Plan* out) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h >= 1 && w >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(c < (int64_t(1) << 31) && d < (int64_t(1) << 31) && h < (int64_t(1) << 31) &&
                        w < (int64_t(1) << 31),
                    "each dimension must fit in int32");
  MEDNEXT_CHECK_ARG(h * w < (int64_t(1) << 40), "plane too large");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  MEDNEXT_CHECK_ARG(tile_w == 4 || tile_w == 8 || tile_w == 16 || tile_w == 32 || tile_w == 64,
                    "tile_w must be 4, 8, 16, 32 or 64");
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  DwGeom g{};
  g.C = static_cast<int>(c);
  g.D = static_cast<int>(d);
  g.H = static_cast<int>(h);
  g.W = static_cast<int>(w);
  g.TD = static_cast<int>(depth_chunk < d ? depth_chunk : d);
  g.TWt = tile_w / 4;
  int tht = kMaxThreads / g.TWt;
  const int need = static_cast<int>(cdiv(h, kRH));
  if (tht > need) tht = need;
  g.THt = tht;
  g.nDc = static_cast<int>(cdiv(d, g.TD));
  g.nHt = static_cast<int>(cdiv(h, kRH * g.THt));
  g.nWt = static_cast<int>(cdiv(w, 4 * g.TWt));
  const int used = g.TWt * g.THt;
  out->threads = static_cast<int>(cdiv(used, 64) * 64);
  const int p = k / 2;
  out->lds_bytes = static_cast<size_t>(kRH * g.THt + 2 * p) * (4 * g.TWt + 8) * acc_bytes;
  MEDNEXT_CHECK_ARG(out->lds_bytes <= 64 * 1024, "tile needs more than 64 KiB of LDS");
  const int64_t splits = n * g.nDc * g.nHt * g.nWt;
  out->blocks = splits * c;
  MEDNEXT_CHECK_ARG(out->blocks < (int64_t(1) << 31), "grid too large");
  out->splits = static_cast<int>(splits);
  out->g = g;
  return MEDNEXT_STATUS_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <typename T, int K, bool FLIP>
int launch_stencil_k(const void* x, const void* wt, const void* bias, void* y, const Plan& pl,
                     bool vec, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(pl.blocks));
  const dim3 block(pl.threads);
  auto px = static_cast<const T*>(x);
  auto pw = static_cast<const T*>(wt);
  auto pb = static_cast<const T*>(bias);
  auto py = static_cast<T*>(y);
  if (vec) {
    if (bias)
      hipLaunchKernelGGL((dw_stencil_kernel<T, Acc, K, FLIP, true, true>), grid, block,
                         pl.lds_bytes, st, px, pw, pb, py, pl.g);
    else
      hipLaunchKernelGGL((dw_stencil_kernel<T, Acc, K, FLIP, true, false>), grid, block,
                         pl.lds_bytes, st, px, pw, pb, py, pl.g);
  } else {
    if (bias)
      hipLaunchKernelGGL((dw_stencil_kernel<T, Acc, K, FLIP, false, true>), grid, block,
                         pl.lds_bytes, st, px, pw, pb, py, pl.g);
    else
      hipLaunchKernelGGL((dw_stencil_kernel<T, Acc, K, FLIP, false, false>), grid, block,
                         pl.lds_bytes, st, px, pw, pb, py, pl.g);
  }
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T, bool FLIP>
int launch_stencil(const void* x, const void* wt, const void* bias, void* y, const Plan& pl,
                   int k, bool vec, hipStream_t st) {
  switch (k) {
    case 1: return launch_stencil_k<T, 1, FLIP>(x, wt, bias, y, pl, vec, st);
    case 3: return launch_stencil_k<T, 3, FLIP>(x, wt, bias, y, pl, vec, st);
    default: return launch_stencil_k<T, 5, FLIP>(x, wt, bias, y, pl, vec, st);
  }
}

int acc_bytes_of(int dtype) { return dtype == MEDNEXT_DTYPE_F64 ? 8 : 4; }

bool dtype_ok(int dtype) {
  return dtype == MEDNEXT_DTYPE_F32 || dtype == MEDNEXT_DTYPE_F64 || dtype == MEDNEXT_DTYPE_F16 ||
         dtype == MEDNEXT_DTYPE_BF16;
}

template <bool FLIP>
int stencil_entry(const void* x, const void* weight, const void* bias, void* y, int64_t n,
                  int64_t c, int64_t d, int64_t h, int64_t w, int32_t k, int32_t dtype,
                  int32_t engine, int32_t tile_w, int32_t depth_chunk, void* stream) {
  MEDNEXT_CHECK_ARG(x != nullptr && weight != nullptr && y != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG((reinterpret_cast<uintptr_t>(weight) & 3u) == 0,
                    "weight must be 4-byte aligned");
  MEDNEXT_CHECK_ARG(engine == MEDNEXT_ENGINE_VALU || engine == MEDNEXT_ENGINE_MFMA || engine == MEDNEXT_ENGINE_VOLUME,
                    "engine must be MEDNEXT_ENGINE_VALU, MEDNEXT_ENGINE_MFMA or MEDNEXT_ENGINE_VOLUME");
  auto s = static_cast<hipStream_t>(stream);
  if (engine == MEDNEXT_ENGINE_VOLUME) {
    return dw_volume_stencil(x, weight, bias, y, n, c, d, h, w, k, dtype, FLIP, tile_w, depth_chunk, s);
  }
  if (engine == MEDNEXT_ENGINE_MFMA) {
    MEDNEXT_CHECK_ARG(dtype == MEDNEXT_DTYPE_BF16, "the MFMA engine is bf16 only");
    MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h < (int64_t(1) << 31) &&
                          c < (int64_t(1) << 31) && d < (int64_t(1) << 31),
                      "shape out of range");
    MEDNEXT_CHECK_ARG(aligned16(x) && aligned16(y), "MFMA engine needs 16-byte aligned tensors");
    return dw_mfma_stencil(x, weight, bias, y, n, c, d, h, w, k, FLIP, tile_w, depth_chunk, s);
  }
  Plan pl;
  int st = make_plan(n, c, d, h, w, k, acc_bytes_of(dtype), tile_w, depth_chunk, &pl);
  if (st != MEDNEXT_STATUS_OK) return st;
  const bool vec = (w % 4 == 0) && aligned16(x) && aligned16(y);
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: return launch_stencil<float, FLIP>(x, weight, bias, y, pl, k, vec, s);
    case MEDNEXT_DTYPE_F64: return launch_stencil<double, FLIP>(x, weight, bias, y, pl, k, vec, s);
    case MEDNEXT_DTYPE_F16: return launch_stencil<f16_t, FLIP>(x, weight, bias, y, pl, k, vec, s);
    default: return launch_stencil<bf16_t, FLIP>(x, weight, bias, y, pl, k, vec, s);
  }
}

template <typename T, int K>
int launch_wgrad_k(const void* x, const void* dy, void* dw, void* db, void* ws, const Plan& pl,
                   bool vec, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(pl.blocks));
  const dim3 block(pl.threads);
  auto px = static_cast<const T*>(x);
  auto pdy = static_cast<const T*>(dy);
  auto part = static_cast<Acc*>(ws);
  if (vec)
    hipLaunchKernelGGL((dw_wgrad_kernel<T, Acc, K, true>), grid, block, pl.lds_bytes, st, px, pdy,
                       part, pl.g, pl.splits);
  else
    hipLaunchKernelGGL((dw_wgrad_kernel<T, Acc, K, false>), grid, block, pl.lds_bytes, st, px,
                       pdy, part, pl.g, pl.splits);
  MEDNEXT_CHECK_LAUNCH();
  return launch_finish<T, Acc>(part, dw, db, pl.g.C, pl.splits, K * K * K, st);
}

template <typename T>
int launch_wgrad(const void* x, const void* dy, void* dw, void* db, void* ws, const Plan& pl, int k,
                 bool vec, hipStream_t st) {
  switch (k) {
    case 1: return launch_wgrad_k<T, 1>(x, dy, dw, db, ws, pl, vec, st);
    case 3: return launch_wgrad_k<T, 3>(x, dy, dw, db, ws, pl, vec, st);
    default: return launch_wgrad_k<T, 5>(x, dy, dw, db, ws, pl, vec, st);
  }
}


// ------------------------------------------------------------------ stride 2
//
// The MedNeXt down block's depthwise conv (stride 2, padding k/2) and the up
// block's depthwise transposed conv (stride 2, padding k/2, no output
// padding) are three index maps between a full-resolution ("big") tensor and
// a half-resolution ("small") one, per channel and with zero padding:
//   gather   small[o] = b + sum_t w[t] * big[2o + t - P]        (down forward;
//                                                                 up input-grad)
//   scatter  big[i]   = b + sum_{o,t: 2o+t-P = i} w[t] * small[o] (down input-grad;
//                                                                 up forward)
//   reduce   dW[t] = sum_o big[2o + t - P] * small[o], dB = sum_o small[o]
//            (down weight-grad with big = x, small = dy; up weight-grad with
//            big = dy, small = x)
// They carry ~k^3/8 FLOP per big element, so they are VALU kernels bound by
// memory; accumulation is fp32 (fp64 for fp64 tensors).
//
// Work decomposition: a wave owns one "task" at a time, a run of up to 64
// consecutive elements of one row of the lane domain: small rows for gather
// and reduce; for scatter, rows of 2x2x2 big-voxel cells, so that every lane
// of every task uses the same taps. Narrow rows pack 64 / Wl rows into one
// task. Tasks never cross a channel slab, so the channel and its weights are
// wave-uniform; task -> row decoding uses 32-bit multiply-high division. All
// loads go through per-slab buffer resources with masked lanes pointed out of
// range (they read zero), so a task issues its loads without branches. A wave
// walks a contiguous run of tasks, so big rows shared by neighbouring output
// rows hit in L1/L2.

// n / d for n < 2^31 by multiply-high (the round-up method: Granlund and
// Montgomery, "Division by invariant integers using multiplication", 1994).
struct FastDiv {
  uint32_t d, m, s;
};

FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
  return FastDiv{d, static_cast<uint32_t>(m), s};
}

__device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) { return (__umulhi(n, f.m) + n) >> f.s; }

struct S2Dims {
  int C;
  int Db, Hb, Wb;  // big
  int Ds, Hs, Ws;  // small
  int Wd;          // lane-domain row width (columns, or column pairs for scatter)
  uint32_t rows;   // lane-domain rows per slab
  int Wl, lshift;  // lanes per row (power of two <= 64) and its log2
  int rpw, nseg;   // rows per task, tasks per row
  uint32_t tpc;    // tasks per (n, c) slab
  uint32_t tasks;  // tasks over the launch
  uint32_t per;    // tasks per wave (gather / scatter) or per workgroup (reduce)
  FastDiv f_tpc, f_nseg, f_Hd, f_C;
};

struct TaskPos {
  uint32_t nc;
  int c;
  int d, h, col;  // lane-domain plane, row, column
  bool valid;
};

__device__ inline TaskPos task_pos(const S2Dims& g, uint32_t nc, uint32_t t, int lane) {
  TaskPos p;
  p.nc = nc;
  p.c = static_cast<int>(nc - fdiv(nc, g.f_C) * static_cast<uint32_t>(g.C));
  const uint32_t rt = fdiv(t, g.f_nseg);
  const uint32_t seg = t - rt * static_cast<uint32_t>(g.nseg);
  const uint32_t row = rt * static_cast<uint32_t>(g.rpw) + static_cast<uint32_t>(lane >> g.lshift);
  p.col = static_cast<int>(seg) * g.Wl + (lane & (g.Wl - 1));
  p.valid = row < g.rows && p.col < g.Wd;
  const uint32_t r = row < g.rows ? row : 0u;
  const uint32_t d = fdiv(r, g.f_Hd);
  p.d = static_cast<int>(d);
  p.h = static_cast<int>(r - d * g.f_Hd.d);
  return p;
}

template <typename T, typename Acc, int K>
__device__ inline void load_taps(const T* __restrict__ w, int c, Acc (&wv)[K * K * K]) {
  const T* wc = w + static_cast<int64_t>(c) * K * K * K;
#pragma unroll
  for (int t = 0; t < K * K * K; ++t) wv[t] = Cvt<T, Acc>::load(wc[t]);
}

template <typename T>
__device__ inline __amdgpu_buffer_rsrc_t s2_rsrc(const T* base, uint32_t slab, int64_t vol) {
  return slab_rsrc(base + slab * vol, static_cast<uint32_t>(vol * static_cast<int64_t>(sizeof(T))));
}

template <typename T, typename Acc, int K, bool BIAS>
__global__ __launch_bounds__(256) void s2_gather_kernel(const T* __restrict__ big, const T* __restrict__ w,
                                                        const T* __restrict__ b, T* __restrict__ out, S2Dims g) {
  constexpr int P = K / 2;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * 4u + static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
  const uint32_t t0 = wave * g.per;
  const uint32_t t1 = min(t0 + g.per, g.tasks);
  const int64_t big_vol = static_cast<int64_t>(g.Db) * g.Hb * g.Wb;
  const int64_t small_vol = static_cast<int64_t>(g.Ds) * g.Hs * g.Ws;
  Acc wv[K * K * K];
  Acc bias = Acc(0);
  int wc = -1;
  for (uint32_t task = t0; task < t1; ++task) {
    const uint32_t nc = fdiv(task, g.f_tpc);
    const TaskPos p = task_pos(g, nc, task - nc * g.tpc, lane);
    if (p.c != wc) {
      load_taps<T, Acc, K>(w, p.c, wv);
      if (BIAS) bias = Cvt<T, Acc>::load(b[p.c]);
      wc = p.c;
    }
    const __amdgpu_buffer_rsrc_t br = s2_rsrc(big, nc, big_vol);
    Acc v[K * K * K];
#pragma unroll
    for (int kd = 0; kd < K; ++kd) {
      const int id = 2 * p.d + kd - P;
      const bool okd = p.valid && static_cast<unsigned>(id) < static_cast<unsigned>(g.Db);
#pragma unroll
      for (int kh = 0; kh < K; ++kh) {
        const int ih = 2 * p.h + kh - P;
        const bool okh = okd && static_cast<unsigned>(ih) < static_cast<unsigned>(g.Hb);
        const int rowoff = (id * g.Hb + ih) * g.Wb;
#pragma unroll
        for (int kw = 0; kw < K; ++kw) {
          const int iw = 2 * p.col + kw - P;
          const bool ok = okh && static_cast<unsigned>(iw) < static_cast<unsigned>(g.Wb);
          v[(kd * K + kh) * K + kw] = BufIo<T>::ld(br, boff<T>(ok, rowoff + iw));
        }
      }
    }
    Acc acc = bias;
#pragma unroll
    for (int t = 0; t < K * K * K; ++t) acc += wv[t] * v[t];
    const __amdgpu_buffer_rsrc_t orr = s2_rsrc(out, nc, small_vol);
    BufIo<T>::st(orr, boff<T>(p.valid, (p.d * g.Hs + p.h) * g.Ws + p.col), acc);
  }
}

// Scatter by 2x2x2 cells: lane (jd, jh, m) of the cell domain produces big
// voxels (2jd + ed, 2jh + eh, 2m + ew), e in {0, 1}. Tap k reaches big index
// 2j + e from small index j + a with a = (e + P - k) / 2 when e + P - k is
// even, so the cell reads the small block j + a, a in [-(P / 2), (P + 1) / 2],
// and every (e, a) -> k pairing is fixed at compile time.
template <typename T, typename Acc, int K, bool BIAS>
__global__ __launch_bounds__(256) void s2_scatter_kernel(const T* __restrict__ small, const T* __restrict__ w,
                                                         const T* __restrict__ b, T* __restrict__ out, S2Dims g) {
  constexpr int P = K / 2;
  constexpr int AMIN = -(P / 2), AMAX = (P + 1) / 2, NA = AMAX - AMIN + 1;
  const int lane = threadIdx.x & 63;
  const uint32_t wave = blockIdx.x * 4u + static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
  const uint32_t t0 = wave * g.per;
  const uint32_t t1 = min(t0 + g.per, g.tasks);
  const int64_t big_vol = static_cast<int64_t>(g.Db) * g.Hb * g.Wb;
  const int64_t small_vol = static_cast<int64_t>(g.Ds) * g.Hs * g.Ws;
  Acc wv[K * K * K];
  Acc bias = Acc(0);
  int wc = -1;
  for (uint32_t task = t0; task < t1; ++task) {
    const uint32_t nc = fdiv(task, g.f_tpc);
    const TaskPos p = task_pos(g, nc, task - nc * g.tpc, lane);
    if (p.c != wc) {
      load_taps<T, Acc, K>(w, p.c, wv);
      if (BIAS) bias = Cvt<T, Acc>::load(b[p.c]);
      wc = p.c;
    }
    const __amdgpu_buffer_rsrc_t sr = s2_rsrc(small, nc, small_vol);
    Acc s[NA][NA][NA];
#pragma unroll
    for (int ad = 0; ad < NA; ++ad) {
      const int sd = p.d + AMIN + ad;
      const bool okd = p.valid && static_cast<unsigned>(sd) < static_cast<unsigned>(g.Ds);
#pragma unroll
      for (int ah = 0; ah < NA; ++ah) {
        const int sh = p.h + AMIN + ah;
        const bool okh = okd && static_cast<unsigned>(sh) < static_cast<unsigned>(g.Hs);
        const int rowoff = (sd * g.Hs + sh) * g.Ws;
#pragma unroll
        for (int aw = 0; aw < NA; ++aw) {
          const int sw = p.col + AMIN + aw;
          const bool ok = okh && static_cast<unsigned>(sw) < static_cast<unsigned>(g.Ws);
          s[ad][ah][aw] = BufIo<T>::ld(sr, boff<T>(ok, rowoff + sw));
        }
      }
    }
    const __amdgpu_buffer_rsrc_t orr = s2_rsrc(out, nc, big_vol);
#pragma unroll
    for (int ed = 0; ed < 2; ++ed) {
      const int bd = 2 * p.d + ed;
#pragma unroll
      for (int eh = 0; eh < 2; ++eh) {
        const int bh = 2 * p.h + eh;
#pragma unroll
        for (int ew = 0; ew < 2; ++ew) {
          const int bw = 2 * p.col + ew;
          Acc acc = bias;
#pragma unroll
          for (int ad = 0; ad < NA; ++ad) {
            const int kd = ed + P - 2 * (AMIN + ad);
            if (kd < 0 || kd >= K) continue;
#pragma unroll
            for (int ah = 0; ah < NA; ++ah) {
              const int kh = eh + P - 2 * (AMIN + ah);
              if (kh < 0 || kh >= K) continue;
#pragma unroll
              for (int aw = 0; aw < NA; ++aw) {
                const int kw = ew + P - 2 * (AMIN + aw);
                if (kw < 0 || kw >= K) continue;
                acc += wv[(kd * K + kh) * K + kw] * s[ad][ah][aw];
              }
            }
          }
          const bool ok = p.valid && bd < g.Db && bh < g.Hb && bw < g.Wb;
          BufIo<T>::st(orr, boff<T>(ok, (bd * g.Hb + bh) * g.Wb + bw), acc);
        }
      }
    }
  }
}

// One workgroup per (n, c, run of tasks); its four waves split the run. Per
// workgroup fp32 (fp64) partials [C][K^3 + 1][splits], split = n * bpc + j,
// summed by the fixed-order finish kernel.
template <typename T, typename Acc, int K>
__global__ __launch_bounds__(256) void s2_wgrad_kernel(const T* __restrict__ big, const T* __restrict__ small,
                                                       Acc* __restrict__ partial, S2Dims g, int bpc, int splits) {
  constexpr int P = K / 2;
  constexpr int K3 = K * K * K;
  __shared__ Acc red[4][K3 + 1];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t nc = blockIdx.x / static_cast<uint32_t>(bpc);
  const uint32_t j = blockIdx.x - nc * static_cast<uint32_t>(bpc);
  const uint32_t b0 = j * g.per;
  const uint32_t b1 = min(b0 + g.per, g.tpc);
  const uint32_t q = (b1 - b0 + 3u) / 4u;
  const uint32_t t0 = min(b0 + wave * q, b1);
  const uint32_t t1 = min(t0 + q, b1);
  const int64_t big_vol = static_cast<int64_t>(g.Db) * g.Hb * g.Wb;
  const int64_t small_vol = static_cast<int64_t>(g.Ds) * g.Hs * g.Ws;
  const __amdgpu_buffer_rsrc_t br = s2_rsrc(big, nc, big_vol);
  const __amdgpu_buffer_rsrc_t sr = s2_rsrc(small, nc, small_vol);
  Acc acc[K3 + 1];
#pragma unroll
  for (int t = 0; t <= K3; ++t) acc[t] = Acc(0);
  for (uint32_t t = t0; t < t1; ++t) {
    const TaskPos p = task_pos(g, nc, t, lane);
    const Acc s = BufIo<T>::ld(sr, boff<T>(p.valid, (p.d * g.Hs + p.h) * g.Ws + p.col));
    Acc v[K3];
#pragma unroll
    for (int kd = 0; kd < K; ++kd) {
      const int id = 2 * p.d + kd - P;
      const bool okd = p.valid && static_cast<unsigned>(id) < static_cast<unsigned>(g.Db);
#pragma unroll
      for (int kh = 0; kh < K; ++kh) {
        const int ih = 2 * p.h + kh - P;
        const bool okh = okd && static_cast<unsigned>(ih) < static_cast<unsigned>(g.Hb);
        const int rowoff = (id * g.Hb + ih) * g.Wb;
#pragma unroll
        for (int kw = 0; kw < K; ++kw) {
          const int iw = 2 * p.col + kw - P;
          const bool ok = okh && static_cast<unsigned>(iw) < static_cast<unsigned>(g.Wb);
          v[(kd * K + kh) * K + kw] = BufIo<T>::ld(br, boff<T>(ok, rowoff + iw));
        }
      }
    }
    acc[K3] += s;
#pragma unroll
    for (int t2 = 0; t2 < K3; ++t2) acc[t2] += v[t2] * s;
  }
#pragma unroll
  for (int t = 0; t <= K3; ++t) {
    const Acc tot = wave_sum(acc[t]);
    if (lane == 0) red[wave][t] = tot;
  }
  __syncthreads();
  const int64_t n = nc / static_cast<uint32_t>(g.C);
  const int c = static_cast<int>(nc - n * g.C);
  const int64_t split = n * bpc + j;
  for (int t = threadIdx.x; t <= K3; t += 256) {
    partial[(static_cast<int64_t>(c) * (K3 + 1) + t) * splits + split] = ((red[0][t] + red[1][t]) + red[2][t]) + red[3][t];
  }
}

constexpr int kS2MaxWaves = 16384;  // gather / scatter: ~8 resident waves per SIMD over two rounds
constexpr int kS2WgradBlocks = 2048;

enum S2Domain { kSmallDomain = 0, kBigCellDomain = 1 };

// Validates the shapes and lays out the lane domain. Every index the kernels
// form stays below 2^31: per-slab volumes, rows and task counts are checked.
int s2_plan(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k,
            int dtype, S2Domain dom, S2Dims* g) {
  MEDNEXT_CHECK_ARG(dtype_ok(dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && db >= 1 && hb >= 1 && wb >= 1 && ds >= 1 && hs >= 1 && ws >= 1,
                    "shape must be positive");
  const int64_t lim = int64_t(1) << 31;
  const int64_t esz = acc_bytes_of(dtype) == 8 ? 8 : (dtype == MEDNEXT_DTYPE_F32 ? 4 : 2);
  MEDNEXT_CHECK_ARG(db * hb * wb * esz < lim && ds * hs * ws * esz < lim,
                    "each (n, c) slab must be smaller than 2 GiB");
  MEDNEXT_CHECK_ARG(n * c < lim, "n * c must be below 2^31");
  g->C = static_cast<int>(c);
  g->Db = static_cast<int>(db);
  g->Hb = static_cast<int>(hb);
  g->Wb = static_cast<int>(wb);
  g->Ds = static_cast<int>(ds);
  g->Hs = static_cast<int>(hs);
  g->Ws = static_cast<int>(ws);
  const int64_t dd = dom == kSmallDomain ? ds : cdiv(db, 2);
  const int64_t hd = dom == kSmallDomain ? hs : cdiv(hb, 2);
  const int64_t wd = dom == kSmallDomain ? ws : cdiv(wb, 2);
  int wl = 1, lshift = 0;
  while (wl < 64 && wl < wd) {
    wl *= 2;
    ++lshift;
  }
  g->Wd = static_cast<int>(wd);
  g->rows = static_cast<uint32_t>(dd * hd);
  g->Wl = wl;
  g->lshift = lshift;
  g->rpw = 64 / wl;
  g->nseg = static_cast<int>(cdiv(wd, wl));
  const int64_t tpc = cdiv(dd * hd, g->rpw) * g->nseg;
  MEDNEXT_CHECK_ARG(n * c * tpc < lim, "too many row tasks");
  g->tpc = static_cast<uint32_t>(tpc);
  g->tasks = static_cast<uint32_t>(n * c * tpc);
  g->f_tpc = make_fastdiv(g->tpc);
  g->f_nseg = make_fastdiv(static_cast<uint32_t>(g->nseg));
  g->f_Hd = make_fastdiv(static_cast<uint32_t>(hd));
  g->f_C = make_fastdiv(static_cast<uint32_t>(c));
  g->per = 1;
  return MEDNEXT_STATUS_OK;
}

// Gather / scatter grid: up to kS2MaxWaves waves, each walking `per` tasks.
unsigned s2_map_blocks(S2Dims* g) {
  const int64_t waves = std::min<int64_t>(g->tasks, kS2MaxWaves);
  g->per = static_cast<uint32_t>(cdiv(g->tasks, waves));
  return static_cast<unsigned>(cdiv(cdiv(g->tasks, g->per), 4));
}

// Reduce grid: ~kS2WgradBlocks workgroups, at least 8 tasks each.
void s2_wgrad_split(int64_t n, S2Dims* g, int* bpc) {
  const int64_t want = cdiv(int64_t(kS2WgradBlocks), n * g->C);
  const int64_t cap = cdiv(g->tpc, int64_t(8));
  const int64_t b = std::max<int64_t>(1, std::min(want, cap));
  g->per = static_cast<uint32_t>(cdiv(g->tpc, b));
  *bpc = static_cast<int>(cdiv(g->tpc, g->per));
}

template <typename T, int K, bool GATHER>
int launch_s2_map_k(const void* in, const void* w, const void* b, void* out, S2Dims g, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const unsigned blocks = s2_map_blocks(&g);
  auto pi = static_cast<const T*>(in);
  auto pw = static_cast<const T*>(w);
  auto pb = static_cast<const T*>(b);
  auto po = static_cast<T*>(out);
  if (GATHER) {
    if (b != nullptr)
      hipLaunchKernelGGL((s2_gather_kernel<T, Acc, K, true>), dim3(blocks), dim3(256), 0, st, pi, pw, pb, po, g);
    else
      hipLaunchKernelGGL((s2_gather_kernel<T, Acc, K, false>), dim3(blocks), dim3(256), 0, st, pi, pw, pb, po, g);
  } else {
    if (b != nullptr)
      hipLaunchKernelGGL((s2_scatter_kernel<T, Acc, K, true>), dim3(blocks), dim3(256), 0, st, pi, pw, pb, po, g);
    else
      hipLaunchKernelGGL((s2_scatter_kernel<T, Acc, K, false>), dim3(blocks), dim3(256), 0, st, pi, pw, pb, po, g);
  }
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

// bf16 stride-2 maps whose big plane is too large for the band kernels
// (small plane above 256 positions) run on the matrix-core stencil / weight
// gradient when the shape is the down block's (even big dims, W % 32 == 0).
bool s2_mfma_chosen(int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, int dtype) {
  return dtype == MEDNEXT_DTYPE_BF16 && hs * ws > 256 && dw_mfma_s2_supported(db, hb, wb, ds, hs, ws, k);
}

template <bool GATHER>
int s2_map_entry(const void* in, const void* w, const void* b, void* out, int64_t n, int64_t c, int64_t db,
                 int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int32_t k, int32_t dtype, void* stream) {
  MEDNEXT_CHECK_ARG(in != nullptr && w != nullptr && out != nullptr, "null tensor pointer");
  S2Dims g;
  if (int st = s2_plan(n, c, db, hb, wb, ds, hs, ws, k, dtype, GATHER ? kSmallDomain : kBigCellDomain, &g))
    return st;
  auto s = static_cast<hipStream_t>(stream);
  if (s2_mfma_chosen(db, hb, wb, ds, hs, ws, k, dtype)) {
    return GATHER ? dw_mfma_s2_gather(in, w, b, out, n, c, db, hb, wb, ds, hs, ws, k, s)
                  : dw_mfma_s2_scatter(in, w, b, out, n, c, db, hb, wb, ds, hs, ws, k, s);
  }
  if (GATHER && dw_s2band_chosen(n, c, db, hb, wb, ds, hs, ws, k, dtype))
    return dw_s2band_gather(in, w, b, out, n, c, db, hb, wb, ds, hs, ws, k, dtype, s);
#define MEDNEXT_S2_K(T)                                                          \
  switch (k) {                                                                   \
    case 1: return launch_s2_map_k<T, 1, GATHER>(in, w, b, out, g, s);           \
    case 3: return launch_s2_map_k<T, 3, GATHER>(in, w, b, out, g, s);           \
    default: return launch_s2_map_k<T, 5, GATHER>(in, w, b, out, g, s);          \
  }
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_S2_K(float)
    case MEDNEXT_DTYPE_F64: MEDNEXT_S2_K(double)
    case MEDNEXT_DTYPE_F16: MEDNEXT_S2_K(f16_t)
    default: MEDNEXT_S2_K(bf16_t)
  }
#undef MEDNEXT_S2_K
}

template <typename T, int K>
int launch_s2_wgrad_k(const void* big, const void* small, void* dw, void* dbias, void* ws, const S2Dims& g,
                      int64_t n, int bpc, hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const int splits = static_cast<int>(n * bpc);
  auto part = static_cast<Acc*>(ws);
  hipLaunchKernelGGL((s2_wgrad_kernel<T, Acc, K>), dim3(static_cast<unsigned>(n * g.C * bpc)), dim3(256), 0, st,
                     static_cast<const T*>(big), static_cast<const T*>(small), part, g, bpc, splits);
  MEDNEXT_CHECK_LAUNCH();
  return launch_finish<T, Acc>(part, dw, dbias, g.C, splits, K * K * K, st);
}

}  // namespace
}  // namespace mednext

using namespace mednext;

extern "C" int32_t mednext_depthwise3d_fwd(const void* x, const void* weight, const void* bias,
                                           void* y, int64_t n, int64_t c, int64_t d, int64_t h,
                                           int64_t w, int32_t kernel_size, int32_t dtype,
                                           int32_t engine, int32_t tile_w, int32_t depth_chunk,
                                           void* stream) {
  return stencil_entry<false>(x, weight, bias, y, n, c, d, h, w, kernel_size, dtype, engine,
                              tile_w, depth_chunk, stream);
}

extern "C" int32_t mednext_depthwise3d_dgrad(const void* grad_output, const void* weight,
                                             void* grad_input, int64_t n, int64_t c, int64_t d,
                                             int64_t h, int64_t w, int32_t kernel_size,
                                             int32_t dtype, int32_t engine, int32_t tile_w,
                                             int32_t depth_chunk, void* stream) {
  return stencil_entry<true>(grad_output, weight, nullptr, grad_input, n, c, d, h, w, kernel_size,
                             dtype, engine, tile_w, depth_chunk, stream);
}

extern "C" int32_t mednext_depthwise3d_dgrad_acc(const void* grad_output, const void* weight,
                                                 const void* accumulate, void* grad_input, int64_t n, int64_t c,
                                                 int64_t d, int64_t h, int64_t w, int32_t kernel_size,
                                                 int32_t dtype, int32_t engine, int32_t tile_w,
                                                 int32_t depth_chunk, void* stream) {
  MEDNEXT_CHECK_ARG(grad_output != nullptr && weight != nullptr && accumulate != nullptr && grad_input != nullptr,
                    "null tensor pointer");
  MEDNEXT_CHECK_ARG(engine == MEDNEXT_ENGINE_MFMA && dtype == MEDNEXT_DTYPE_BF16 &&
                        (kernel_size == 3 || kernel_size == 5),
                    "the accumulating input gradient runs the bf16 k = 3 / 5 matrix-core kernels");
  MEDNEXT_CHECK_ARG((reinterpret_cast<uintptr_t>(weight) & 3u) == 0, "weight must be 4-byte aligned");
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h < (int64_t(1) << 31) && c < (int64_t(1) << 31) &&
                        d < (int64_t(1) << 31),
                    "shape out of range");
  MEDNEXT_CHECK_ARG(aligned16(grad_output) && aligned16(grad_input) && aligned16(accumulate),
                    "MFMA engine needs 16-byte aligned tensors");
  return dw_mfma_stencil(grad_output, weight, nullptr, grad_input, n, c, d, h, w, kernel_size, true, tile_w,
                         depth_chunk, static_cast<hipStream_t>(stream), accumulate);
}

extern "C" size_t mednext_depthwise3d_wgrad_workspace_bytes(int64_t n, int64_t c, int64_t d,
                                                            int64_t h, int64_t w,
                                                            int32_t kernel_size, int32_t dtype,
                                                            int32_t engine, int32_t tile_w,
                                                            int32_t depth_chunk) {
  if (!dtype_ok(dtype)) return 0;
  const int64_t k3 = int64_t(kernel_size) * kernel_size * kernel_size;
  if (engine == MEDNEXT_ENGINE_MFMA) {
    if (dtype != MEDNEXT_DTYPE_BF16) return 0;
    const int splits = dw_mfma_wgrad_splits(n, c, d, h, w, kernel_size, tile_w, depth_chunk);
    if (splits <= 0) return 0;
    return static_cast<size_t>(c * splits * (k3 + 1) * 4);
  }
  if (engine == MEDNEXT_ENGINE_VOLUME) {
    const int splits = dw_volume_wgrad_splits(n, c, d, h, w, kernel_size, dtype, tile_w, depth_chunk);
    if (splits <= 0) return 0;
    return static_cast<size_t>(c * splits * (k3 + 1) * acc_bytes_of(dtype));
  }
  if (engine != MEDNEXT_ENGINE_VALU) return 0;
  Plan pl;
  if (make_plan(n, c, d, h, w, kernel_size, acc_bytes_of(dtype), tile_w, depth_chunk, &pl) !=
      MEDNEXT_STATUS_OK)
    return 0;
  return static_cast<size_t>(c * pl.splits * (k3 + 1) * acc_bytes_of(dtype));
}

extern "C" int32_t mednext_depthwise3d_wgrad(const void* x, const void* grad_output,
                                             void* grad_weight, void* grad_bias, void* workspace,
                                             size_t workspace_bytes, int64_t n, int64_t c,
                                             int64_t d, int64_t h, int64_t w, int32_t kernel_size,
                                             int32_t dtype, int32_t engine, int32_t tile_w,
                                             int32_t depth_chunk, void* stream) {
  MEDNEXT_CHECK_ARG(x != nullptr && grad_output != nullptr && grad_weight != nullptr,
                    "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(engine == MEDNEXT_ENGINE_VALU || engine == MEDNEXT_ENGINE_MFMA || engine == MEDNEXT_ENGINE_VOLUME,
                    "engine must be MEDNEXT_ENGINE_VALU, MEDNEXT_ENGINE_MFMA or MEDNEXT_ENGINE_VOLUME");
  const int64_t k3 = int64_t(kernel_size) * kernel_size * kernel_size;
  auto s = static_cast<hipStream_t>(stream);
  if (engine == MEDNEXT_ENGINE_VOLUME) {
    const int splits = dw_volume_wgrad_splits(n, c, d, h, w, kernel_size, dtype, tile_w, depth_chunk);
    if (splits <= 0) {
      // The planner names the reason.
      return dw_volume_wgrad(x, grad_output, nullptr, n, c, d, h, w, kernel_size, dtype, tile_w, depth_chunk, s);
    }
    const size_t need = static_cast<size_t>(c * splits * (k3 + 1) * acc_bytes_of(dtype));
    MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
    int st = dw_volume_wgrad(x, grad_output, workspace, n, c, d, h, w, kernel_size, dtype, tile_w, depth_chunk, s);
    if (st != MEDNEXT_STATUS_OK) return st;
    return finish_partials(dtype, workspace, grad_weight, grad_bias, c, splits, static_cast<int>(k3), s);
  }
  if (engine == MEDNEXT_ENGINE_MFMA) {
    MEDNEXT_CHECK_ARG(dtype == MEDNEXT_DTYPE_BF16, "the MFMA engine is bf16 only");
    MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && c < (int64_t(1) << 31) &&
                          d < (int64_t(1) << 31) && h < (int64_t(1) << 31),
                      "shape out of range");
    MEDNEXT_CHECK_ARG(aligned16(x) && aligned16(grad_output),
                      "MFMA engine needs 16-byte aligned tensors");
    const int splits = dw_mfma_wgrad_splits(n, c, d, h, w, kernel_size, tile_w, depth_chunk);
    MEDNEXT_CHECK_ARG(splits > 0,
                      "MFMA wgrad needs k in {3,5}, W % 32 == 0, H >= 32, tile_w in {32,64,128}");
    const size_t need = static_cast<size_t>(c * splits * (k3 + 1) * 4);
    MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
    auto part = static_cast<float*>(workspace);
    int st = dw_mfma_wgrad(x, grad_output, part, n, c, d, h, w, kernel_size, tile_w, depth_chunk, s);
    if (st != MEDNEXT_STATUS_OK) return st;
    return launch_finish<bf16_t, float>(part, grad_weight, grad_bias, c, splits,
                                        static_cast<int>(k3), s);
  }
  Plan pl;
  int st = make_plan(n, c, d, h, w, kernel_size, acc_bytes_of(dtype), tile_w, depth_chunk, &pl);
  if (st != MEDNEXT_STATUS_OK) return st;
  const size_t need = static_cast<size_t>(c * pl.splits * (k3 + 1) * acc_bytes_of(dtype));
  MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
  const bool vec = (w % 4 == 0) && aligned16(x) && aligned16(grad_output);
  switch (dtype) {
    case MEDNEXT_DTYPE_F32:
      return launch_wgrad<float>(x, grad_output, grad_weight, grad_bias, workspace, pl,
                                 kernel_size, vec, s);
    case MEDNEXT_DTYPE_F64:
      return launch_wgrad<double>(x, grad_output, grad_weight, grad_bias, workspace, pl,
                                  kernel_size, vec, s);
    case MEDNEXT_DTYPE_F16:
      return launch_wgrad<f16_t>(x, grad_output, grad_weight, grad_bias, workspace, pl,
                                 kernel_size, vec, s);
    default:
      return launch_wgrad<bf16_t>(x, grad_output, grad_weight, grad_bias, workspace, pl,
                                  kernel_size, vec, s);
  }
}

// ------------------------------------------- allocation-free weight gradient
//
// mednext_depthwise3d_wgrad_noalloc keeps the fp32 / fp64 partials in this
// library-owned device array instead of a caller workspace. Each GPU holds its
// own copy (at its own address) from the first call on it until the process
// ends; its contents carry over between calls, and every launch overwrites all
// the partial slots it reads, so nothing needs clearing.
constexpr size_t kWgradScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kWgradScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up once per
// device (the host-side name is only a stand-in for the symbol).
int32_t scratch_on_current_device(void* stream, void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) {
    mednext::set_error(std::string("hipGetDevice failed: ") + hipGetErrorString(err));
    return MEDNEXT_STATUS_LAUNCH_ERROR;
  }
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (err != hipSuccess) {
      mednext::set_error(std::string("hipStreamGetDevice failed: ") + hipGetErrorString(err));
      return MEDNEXT_STATUS_LAUNCH_ERROR;
    }
    MEDNEXT_CHECK_ARG(sdev == dev, "the stream belongs to device " + std::to_string(sdev) +
                                       " but device " + std::to_string(dev) + " is current");
  }
  MEDNEXT_CHECK_ARG(dev >= 0 && dev < kMaxScratchDevices, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr) {
      mednext::set_error(std::string("hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(err));
      return MEDNEXT_STATUS_LAUNCH_ERROR;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MEDNEXT_STATUS_OK;
}
}  // namespace

extern "C" size_t mednext_depthwise3d_wgrad_noalloc_max_bytes(void) { return kWgradScratchBytes; }

extern "C" int32_t mednext_depthwise3d_wgrad_noalloc(const void* x, const void* grad_output, void* grad_weight,
                                                     void* grad_bias, int64_t n, int64_t c, int64_t d, int64_t h,
                                                     int64_t w, int32_t kernel_size, int32_t dtype, int32_t engine,
                                                     int32_t tile_w, int32_t depth_chunk, void* stream) {
  const size_t need = mednext_depthwise3d_wgrad_workspace_bytes(n, c, d, h, w, kernel_size, dtype, engine, tile_w,
                                                                depth_chunk);
  if (need == 0) {
    // Unsupported shape or recipe: the allocating entry point names the reason.
    return mednext_depthwise3d_wgrad(x, grad_output, grad_weight, grad_bias, nullptr, 0, n, c, d, h, w, kernel_size,
                                     dtype, engine, tile_w, depth_chunk, stream);
  }
  MEDNEXT_CHECK_ARG(need <= kWgradScratchBytes,
                    "this shape needs " + std::to_string(need) + " bytes of partials, more than the " +
                        std::to_string(kWgradScratchBytes) + "-byte scratch array of the allocation-free entry point");
  void* ptr = nullptr;
  const int32_t st = scratch_on_current_device(stream, &ptr);
  if (st != MEDNEXT_STATUS_OK) return st;
  return mednext_depthwise3d_wgrad(x, grad_output, grad_weight, grad_bias, ptr, kWgradScratchBytes, n, c, d, h, w,
                                   kernel_size, dtype, engine, tile_w, depth_chunk, stream);
}

extern "C" int32_t mednext_depthwise3d_s2_gather(const void* big, const void* weight, const void* bias,
                                                 void* small_out, int64_t n, int64_t c, int64_t db, int64_t hb,
                                                 int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                                 int32_t kernel_size, int32_t dtype, void* stream) {
  return s2_map_entry<true>(big, weight, bias, small_out, n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype, stream);
}

extern "C" int32_t mednext_depthwise3d_s2_scatter(const void* small, const void* weight, const void* bias,
                                                  void* big_out, int64_t n, int64_t c, int64_t db, int64_t hb,
                                                  int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                                  int32_t kernel_size, int32_t dtype, void* stream) {
  return s2_map_entry<false>(small, weight, bias, big_out, n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype, stream);
}

extern "C" size_t mednext_depthwise3d_s2_wgrad_workspace_bytes(int64_t n, int64_t c, int64_t db, int64_t hb,
                                                               int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                                               int32_t kernel_size, int32_t dtype) {
  S2Dims g;
  if (s2_plan(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype, kSmallDomain, &g) != MEDNEXT_STATUS_OK) return 0;
  const int64_t k3 = int64_t(kernel_size) * kernel_size * kernel_size;
  if (s2_mfma_chosen(db, hb, wb, ds, hs, ws, kernel_size, dtype)) {
    const int64_t splits = dw_mfma_s2_wgrad_splits(n, c, db, hb, wb, ds, hs, ws, kernel_size);
    return static_cast<size_t>(c * splits * (k3 + 1) * sizeof(float));
  }
  if (dw_s2band_chosen(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype)) {
    const int64_t splits = dw_s2band_wgrad_splits(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype);
    return static_cast<size_t>(c * splits * (k3 + 1) * acc_bytes_of(dtype));
  }
  int bpc = 0;
  s2_wgrad_split(n, &g, &bpc);
  return static_cast<size_t>(c * n * bpc * (k3 + 1) * acc_bytes_of(dtype));
}

extern "C" int32_t mednext_depthwise3d_s2_wgrad(const void* big, const void* small, void* grad_weight,
                                                void* grad_bias, void* workspace, size_t workspace_bytes,
                                                int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb,
                                                int64_t ds, int64_t hs, int64_t ws, int32_t kernel_size,
                                                int32_t dtype, void* stream) {
  MEDNEXT_CHECK_ARG(big != nullptr && small != nullptr && grad_weight != nullptr, "null tensor pointer");
  S2Dims g;
  if (int st = s2_plan(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype, kSmallDomain, &g)) return st;
  int bpc = 0;
  s2_wgrad_split(n, &g, &bpc);
  MEDNEXT_CHECK_ARG(n * c * bpc < (int64_t(1) << 31), "grid too large");
  const size_t need =
      mednext_depthwise3d_s2_wgrad_workspace_bytes(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype);
  MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
  auto s = static_cast<hipStream_t>(stream);
  if (s2_mfma_chosen(db, hb, wb, ds, hs, ws, kernel_size, dtype)) {
    const int splits = dw_mfma_s2_wgrad_splits(n, c, db, hb, wb, ds, hs, ws, kernel_size);
    if (int st = dw_mfma_s2_wgrad(big, small, static_cast<float*>(workspace), n, c, db, hb, wb, ds, hs, ws,
                                  kernel_size, s))
      return st;
    return finish_partials(dtype, workspace, grad_weight, grad_bias, c, splits,
                           kernel_size * kernel_size * kernel_size, s);
  }
  if (dw_s2band_chosen(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype)) {
    const int splits = dw_s2band_wgrad_splits(n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype);
    if (int st = dw_s2band_wgrad(big, small, workspace, n, c, db, hb, wb, ds, hs, ws, kernel_size, dtype, s))
      return st;
    return finish_partials(dtype, workspace, grad_weight, grad_bias, c, splits,
                           kernel_size * kernel_size * kernel_size, s);
  }
#define MEDNEXT_S2W_K(T)                                                                            \
  switch (kernel_size) {                                                                            \
    case 1: return launch_s2_wgrad_k<T, 1>(big, small, grad_weight, grad_bias, workspace, g, n, bpc, s); \
    case 3: return launch_s2_wgrad_k<T, 3>(big, small, grad_weight, grad_bias, workspace, g, n, bpc, s); \
    default: return launch_s2_wgrad_k<T, 5>(big, small, grad_weight, grad_bias, workspace, g, n, bpc, s); \
  }
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_S2W_K(float)
    case MEDNEXT_DTYPE_F64: MEDNEXT_S2W_K(double)
    case MEDNEXT_DTYPE_F16: MEDNEXT_S2W_K(f16_t)
    default: MEDNEXT_S2W_K(bf16_t)
  }
#undef MEDNEXT_S2W_K
}
