// Depthwise Conv3d (stride 1, odd cubic kernel, zero "same" padding) on small
// planes: H * W <= 256 elements, the MedNeXt stages at 16^3 and 8^3. Every
// dtype; fp32 accumulation (fp64 for fp64).
//
// At these sizes the tiled kernels leave most lanes idle (a 16 x 16 plane is
// one or two 4-column tiles) and run long serial per-thread chains, so they
// are latency-bound at 30-60 us for 1-4 MB of data. Here one workgroup holds
// whole planes: the zero-padded block of input planes a D-chunk needs, for one
// or several (n, c) slabs (`cpw` of them), is staged in LDS (converted to the
// accumulation type), and the lanes map to consecutive (h, w) positions of a
// plane, so every LDS read of a wave touches consecutive addresses and every
// store is one contiguous run of the output.
//
// Forward / input gradient: a lane owns one (h, w) position and kSeg
// consecutive output planes; per (kh, kw) it reads the kSeg + k - 1 input
// values of its column once and applies all k taps along D to them.
//
// Weight gradient: a lane owns one (h, w) position of one slab and walks its
// column of input planes once; each plane's k * k values meet the k most
// recent grad_output values (a register ring), so all k^3 taps and the bias
// sum accumulate in registers in one pass. The lane sums are reduced per
// slab in a fixed order through LDS (segments of 16 lanes, then segments in
// order) into the same [C][k^3 + 1][splits] partial layout as the other
// weight-gradient kernels, and the shared fixed-order finish kernel sums the
// splits (one per (n, D-chunk)).
#include "common.h"
#include "depthwise_volume.h"

#include <algorithm>

namespace mednext {
namespace {

constexpr int kVolThreads = 256;
constexpr int kSeg = 4;  // output planes per lane (forward / input gradient)

struct VolGeom {
  int C, D, H, W;
  int TD;      // output planes per workgroup (D-chunk)
  int TDp;     // TD rounded up to a multiple of kSeg
  int nDc;     // D-chunks per slab
  int cpw;     // slabs per workgroup
  int64_t slabs;
};

template <typename T, typename Acc>
__device__ inline Acc load_acc(const T* p, int64_t i) {
  return Cvt<T, Acc>::load(p[i]);
}

// Stage the zero-padded input planes [d0 - P, d0 + TDp + P) of `cpw` slabs
// starting at slab0 into lds[s][pd][ph][pw] (pitches (H + 2P) x (W + 2P)).
// A lane owns padded plane positions (consecutive lanes: consecutive
// positions, so the loads of a wave are contiguous runs of a row) and loads
// kFillBatch planes of one position before storing any of them, so a
// workgroup waits for a few memory round trips instead of one per element.
constexpr int kFillBatch = 8;

template <typename T, typename Acc, int P>
__device__ inline void fill_volume(Acc* __restrict__ lds, const T* __restrict__ src, const VolGeom& g,
                                   int64_t slab0, int d0) {
  const int Hp = g.H + 2 * P, Wp = g.W + 2 * P, planes = g.TDp + 2 * P, hwp = Hp * Wp;
  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  for (int e2 = threadIdx.x; e2 < hwp; e2 += kVolThreads) {
    const int ph = e2 / Wp, pw = e2 - ph * Wp;
    const int gh = ph - P, gw = pw - P;
    const bool in_plane = gh >= 0 && gh < g.H && gw >= 0 && gw < g.W;
    for (int s = 0; s < g.cpw; ++s) {
      const int64_t slab = slab0 + s;
      const bool ok = in_plane && slab < g.slabs;
      const int64_t base = ok ? (slab * g.D) * plane + static_cast<int64_t>(gh) * g.W + gw : 0;
      Acc* __restrict__ out = lds + static_cast<int64_t>(s) * planes * hwp + e2;
      for (int pd0 = 0; pd0 < planes; pd0 += kFillBatch) {
        Acc v[kFillBatch];
#pragma unroll
        for (int b = 0; b < kFillBatch; ++b) {
          const int gd = d0 - P + pd0 + b;
          v[b] = (ok && pd0 + b < planes && gd >= 0 && gd < g.D) ? load_acc<T, Acc>(src, base + gd * plane) : Acc(0);
        }
#pragma unroll
        for (int b = 0; b < kFillBatch; ++b) {
          if (pd0 + b < planes) out[(pd0 + b) * hwp] = v[b];
        }
      }
    }
  }
}

template <typename T, typename Acc, int K, bool FLIP, bool BIAS>
__global__ __launch_bounds__(kVolThreads) void dw_volume_stencil_kernel(const T* __restrict__ x,
                                                                        const T* __restrict__ wt,
                                                                        const T* __restrict__ bias,
                                                                        T* __restrict__ y, VolGeom g) {
  constexpr int P = K / 2, K3 = K * K * K, COL = kSeg + K - 1;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Hp = g.H + 2 * P, Wp = g.W + 2 * P;
  const int per_slab = (g.TDp + 2 * P) * Hp * Wp;
  Acc* const ws = xs + g.cpw * per_slab;  // [cpw][K3] taps (flipped for the input gradient)
  Acc* const bs = ws + g.cpw * K3;        // [cpw] bias

  const int dc = static_cast<int>(blockIdx.x % g.nDc);
  const int64_t slab0 = static_cast<int64_t>(blockIdx.x / g.nDc) * g.cpw;
  const int d0 = dc * g.TD;
  const int nd = min(g.TD, g.D - d0);

  fill_volume<T, Acc, P>(xs, x, g, slab0, d0);
  for (int e = threadIdx.x; e < g.cpw * K3; e += kVolThreads) {
    const int s = e / K3, t = e - s * K3;
    const int64_t slab = slab0 + s;
    const int64_t c = slab % g.C;
    ws[e] = slab < g.slabs ? load_acc<T, Acc>(wt, c * K3 + (FLIP ? K3 - 1 - t : t)) : Acc(0);
  }
  if (BIAS) {
    for (int s = threadIdx.x; s < g.cpw; s += kVolThreads) {
      const int64_t slab = slab0 + s;
      bs[s] = slab < g.slabs ? load_acc<T, Acc>(bias, slab % g.C) : Acc(0);
    }
  }
  __syncthreads();

  const int hw = g.H * g.W;
  const int groups = g.TDp / kSeg;
  const int items = g.cpw * groups * hw;
  const int64_t plane = hw;
  for (int item = threadIdx.x; item < items; item += kVolThreads) {
    const int p = item % hw;
    const int rest = item / hw;
    const int grp = rest % groups, s = rest / groups;
    const int64_t slab = slab0 + s;
    const int od0 = grp * kSeg;
    if (slab >= g.slabs || od0 >= nd) continue;
    const int h = p / g.W, w = p - h * g.W;
    const Acc* __restrict__ xv = xs + s * per_slab + (od0 * Hp + h) * Wp + w;
    const Acc* __restrict__ wv = ws + s * K3;
    Acc acc[kSeg];
#pragma unroll
    for (int j = 0; j < kSeg; ++j) acc[j] = BIAS ? bs[s] : Acc(0);
    // One kernel row at a time: unrolling kh as well would keep k^2 * COL
    // loaded values live (k = 5: more registers than a lane has).
#pragma unroll 1
    for (int kh = 0; kh < K; ++kh) {
#pragma unroll
      for (int kw = 0; kw < K; ++kw) {
        Acc col[COL];
#pragma unroll
        for (int i = 0; i < COL; ++i) col[i] = xv[(i * Hp + kh) * Wp + kw];
#pragma unroll
        for (int kd = 0; kd < K; ++kd) {
          const Acc tap = wv[(kd * K + kh) * K + kw];
#pragma unroll
          for (int j = 0; j < kSeg; ++j) acc[j] += tap * col[j + kd];
        }
      }
    }
    T* __restrict__ out = y + (slab * g.D + d0 + od0) * plane + p;
#pragma unroll
    for (int j = 0; j < kSeg; ++j) {
      if (od0 + j < nd) out[j * plane] = Cvt<T, Acc>::store(acc[j]);
    }
  }
}

// Taps reduced per LDS round of the weight gradient (fewer for fp64, whose
// staged planes take twice the LDS) and lanes per first-level segment.
template <typename Acc>
constexpr int red_taps() { return sizeof(Acc) == 8 ? 8 : 16; }
constexpr int kRedSeg = 16;

// Input-plane D-run KDP of the k taps along D accumulated per pass: all of
// them (one pass) unless fp64 accumulators for k = 5 would exceed the lanes'
// registers (then one kd per pass).
template <typename Acc, int K>
constexpr int kd_per_pass() { return sizeof(Acc) == 8 && K == 5 ? 1 : K; }

template <typename T, typename Acc, int K>
__global__ __launch_bounds__(kVolThreads) void dw_volume_wgrad_kernel(const T* __restrict__ x,
                                                                      const T* __restrict__ dy,
                                                                      Acc* __restrict__ partial, VolGeom g,
                                                                      int splits) {
  constexpr int P = K / 2, K2 = K * K, K3 = K2 * K;
  constexpr int KDP = kd_per_pass<Acc, K>();
  constexpr int NACC = KDP * K2 + 1;  // taps of one pass + the bias sum
  constexpr int RT = red_taps<Acc>();
  extern __shared__ __align__(16) unsigned char smem_raw[];
  Acc* const xs = reinterpret_cast<Acc*>(smem_raw);
  const int Hp = g.H + 2 * P, Wp = g.W + 2 * P;
  const int hw = g.H * g.W;
  const int planes = g.TDp + 2 * P;
  const int x_slab = planes * Hp * Wp;
  Acc* const ds = xs + g.cpw * x_slab;          // [cpw][TDp][H][W] grad_output
  Acc* const red = ds + g.cpw * g.TDp * hw;      // [RT][kVolThreads] lane values of one round
  Acc* const segs = red + RT * kVolThreads;      // [RT][kVolThreads / kRedSeg] segment sums

  const int dc = static_cast<int>(blockIdx.x % g.nDc);
  const int64_t slab0 = static_cast<int64_t>(blockIdx.x / g.nDc) * g.cpw;
  const int d0 = dc * g.TD;
  const int nd = min(g.TD, g.D - d0);

  fill_volume<T, Acc, P>(xs, x, g, slab0, d0);
  {
    const int64_t plane = hw;
    for (int p = threadIdx.x; p < hw; p += kVolThreads) {
      for (int s = 0; s < g.cpw; ++s) {
        const int64_t slab = slab0 + s;
        const bool ok = slab < g.slabs;
        const int64_t base = ok ? (slab * g.D + d0) * plane + p : 0;
        Acc* __restrict__ out = ds + static_cast<int64_t>(s) * g.TDp * hw + p;
        for (int od0 = 0; od0 < g.TDp; od0 += kFillBatch) {
          Acc v[kFillBatch];
#pragma unroll
          for (int b = 0; b < kFillBatch; ++b)
            v[b] = (ok && od0 + b < nd) ? load_acc<T, Acc>(dy, base + (od0 + b) * plane) : Acc(0);
#pragma unroll
          for (int b = 0; b < kFillBatch; ++b) {
            if (od0 + b < g.TDp) out[(od0 + b) * hw] = v[b];
          }
        }
      }
    }
  }
  __syncthreads();

  // Lane -> (slab s, position p); lanes past cpw * hw only add zeros.
  const int t = threadIdx.x;
  const int s = t / hw, p = t - s * hw;
  const bool active = s < g.cpw;
  const int h = active ? p / g.W : 0, w = active ? p - h * g.W : 0;
  const Acc* __restrict__ xv = xs + (active ? s : 0) * x_slab + h * Wp + w;
  const Acc* __restrict__ dv = ds + (active ? s : 0) * g.TDp * hw + p;
  // Two-level fixed-order lane sums when slabs start on segment boundaries
  // (H * W % kRedSeg == 0; the 8^3 and 16^3 planes), else one lane per
  // (slab, tap) adds the slab's lanes in order.
  const bool by_segment = hw % kRedSeg == 0;

  // Passes and reduction rounds are unrolled so that every register-array
  // index (accumulator, grad_output ring) is a compile-time constant.
#pragma unroll
  for (int kd0 = 0; kd0 < K; kd0 += KDP) {
    // Input plane pd (padded index) meets grad_output plane pd - kd through tap kd.
    Acc acc[NACC];
#pragma unroll
    for (int i = 0; i < NACC; ++i) acc[i] = Acc(0);
    if (active) {
      Acc ring[K];  // ring[j] = grad_output plane pd - j (zero outside [0, TDp))
#pragma unroll
      for (int j = 0; j < K; ++j) ring[j] = Acc(0);
      for (int pd = 0; pd < planes; ++pd) {
#pragma unroll
        for (int j = K - 1; j > 0; --j) ring[j] = ring[j - 1];
        ring[0] = pd < g.TDp ? dv[pd * hw] : Acc(0);
        if (kd0 == 0) acc[NACC - 1] += ring[0];
#pragma unroll
        for (int kh = 0; kh < K; ++kh)
#pragma unroll
          for (int kw = 0; kw < K; ++kw) {
            const Acc xval = xv[(pd * Hp + kh) * Wp + kw];
#pragma unroll
            for (int j = 0; j < KDP; ++j) acc[(j * K + kh) * K + kw] += xval * ring[kd0 + j];
          }
      }
    }
    // Reduce acc over the lanes of each slab, RT taps per round.
    const int ntaps = kd0 == 0 ? NACC : NACC - 1;
#pragma unroll
    for (int r0 = 0; r0 < NACC; r0 += RT) {
      if (r0 >= ntaps) break;
#pragma unroll
      for (int i = 0; i < NACC; ++i) {
        if (i >= r0 && i < r0 + RT) red[(i - r0) * kVolThreads + t] = acc[i];
      }
      __syncthreads();
      const int nr = min(RT, ntaps - r0);
      if (by_segment) {
        constexpr int NSEG = kVolThreads / kRedSeg;
        for (int e = t; e < nr * NSEG; e += kVolThreads) {
          const int i = e / NSEG, q = e - i * NSEG;
          Acc v = Acc(0);
#pragma unroll
          for (int l = 0; l < kRedSeg; ++l) v += red[i * kVolThreads + q * kRedSeg + l];
          segs[i * NSEG + q] = v;
        }
        __syncthreads();
      }
      for (int e = t; e < g.cpw * nr; e += kVolThreads) {
        const int ss = e / nr, i = e - ss * nr;
        const int64_t slab = slab0 + ss;
        if (slab >= g.slabs) continue;
        Acc v = Acc(0);
        if (by_segment) {
          const int NSEG = kVolThreads / kRedSeg;
          for (int q = ss * hw / kRedSeg; q < (ss + 1) * hw / kRedSeg; ++q) v += segs[i * NSEG + q];
        } else {
          for (int q = ss * hw; q < (ss + 1) * hw; ++q) v += red[i * kVolThreads + q];
        }
        const int ai = r0 + i;
        const int tap = ai == NACC - 1 ? K3 : kd0 * K2 + ai;
        const int64_t c = slab % g.C, n = slab / g.C;
        partial[(c * (K3 + 1) + tap) * splits + n * g.nDc + dc] = v;
      }
      __syncthreads();
    }
  }
}

size_t volume_lds_bytes(const VolGeom& g, int k, int acc_bytes, bool wgrad) {
  const int P = k / 2, k3 = k * k * k, k2 = k * k;
  const size_t x = static_cast<size_t>(g.cpw) * (g.TDp + 2 * P) * (g.H + 2 * P) * (g.W + 2 * P);
  if (!wgrad) return (x + static_cast<size_t>(g.cpw) * (k3 + 1)) * acc_bytes;
  const size_t dys = static_cast<size_t>(g.cpw) * g.TDp * g.H * g.W;
  // One round of lane values plus its segment sums.
  const int rt = acc_bytes == 8 ? 8 : 16;
  const size_t red = static_cast<size_t>(rt) * kVolThreads + static_cast<size_t>(rt) * (kVolThreads / kRedSeg);
  (void)k2;
  return (x + dys + red) * acc_bytes;
}

int volume_plan(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int seg, int depth_chunk,
                bool wgrad, VolGeom* g, size_t* lds) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && d >= 1 && h >= 1 && w >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(k == 1 || k == 3 || k == 5, "kernel_size must be 1, 3 or 5");
  MEDNEXT_CHECK_ARG(h * w <= kVolThreads, "the volume engine takes planes of at most 256 elements (H * W)");
  MEDNEXT_CHECK_ARG(seg == kSeg, "the volume engine's tile_w (output planes per lane) must be 4");
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  MEDNEXT_CHECK_ARG(d < (int64_t(1) << 31) && n * c < (int64_t(1) << 40), "shape out of range");
  const int acc = dtype == MEDNEXT_DTYPE_F64 ? 8 : 4;
  g->C = static_cast<int>(c);
  g->D = static_cast<int>(d);
  g->H = static_cast<int>(h);
  g->W = static_cast<int>(w);
  g->TD = static_cast<int>(std::min<int64_t>(depth_chunk, d));
  g->TDp = static_cast<int>(cdiv(g->TD, kSeg) * kSeg);
  g->nDc = static_cast<int>(cdiv(d, g->TD));
  g->slabs = n * c;
  g->cpw = static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(kVolThreads / (h * w), n * c)));
  // Fewer slabs per workgroup until the staged planes fit 64 KiB of LDS.
  while (g->cpw > 1 && volume_lds_bytes(*g, k, acc, wgrad) > 64 * 1024) --g->cpw;
  *lds = volume_lds_bytes(*g, k, acc, wgrad);
  MEDNEXT_CHECK_ARG(*lds <= 64 * 1024, "depth_chunk too long: the staged planes exceed 64 KiB of LDS");
  const int64_t blocks = cdiv(g->slabs, g->cpw) * g->nDc;
  MEDNEXT_CHECK_ARG(blocks < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

template <typename T, int K, bool FLIP>
int launch_volume_stencil(const void* x, const void* wt, const void* bias, void* y, const VolGeom& g, size_t lds,
                          hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(cdiv(g.slabs, g.cpw) * g.nDc));
  auto px = static_cast<const T*>(x);
  auto pw = static_cast<const T*>(wt);
  auto pb = static_cast<const T*>(bias);
  auto py = static_cast<T*>(y);
  if (bias != nullptr)
    hipLaunchKernelGGL((dw_volume_stencil_kernel<T, Acc, K, FLIP, true>), grid, dim3(kVolThreads), lds, st, px, pw,
                       pb, py, g);
  else
    hipLaunchKernelGGL((dw_volume_stencil_kernel<T, Acc, K, FLIP, false>), grid, dim3(kVolThreads), lds, st, px,
                       pw, pb, py, g);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T, bool FLIP>
int volume_stencil_t(const void* x, const void* wt, const void* bias, void* y, const VolGeom& g, int k, size_t lds,
                     hipStream_t st) {
  switch (k) {
    case 1: return launch_volume_stencil<T, 1, FLIP>(x, wt, bias, y, g, lds, st);
    case 3: return launch_volume_stencil<T, 3, FLIP>(x, wt, bias, y, g, lds, st);
    default: return launch_volume_stencil<T, 5, FLIP>(x, wt, bias, y, g, lds, st);
  }
}

template <typename T>
int volume_wgrad_t(const void* x, const void* dy, void* partial, const VolGeom& g, int k, int splits, size_t lds,
                   hipStream_t st) {
  using Acc = typename AccOf<T>::type;
  const dim3 grid(static_cast<unsigned>(cdiv(g.slabs, g.cpw) * g.nDc));
  auto px = static_cast<const T*>(x);
  auto pd = static_cast<const T*>(dy);
  auto part = static_cast<Acc*>(partial);
  switch (k) {
    case 1:
      hipLaunchKernelGGL((dw_volume_wgrad_kernel<T, Acc, 1>), grid, dim3(kVolThreads), lds, st, px, pd, part, g, splits);
      break;
    case 3:
      hipLaunchKernelGGL((dw_volume_wgrad_kernel<T, Acc, 3>), grid, dim3(kVolThreads), lds, st, px, pd, part, g, splits);
      break;
    default:
      hipLaunchKernelGGL((dw_volume_wgrad_kernel<T, Acc, 5>), grid, dim3(kVolThreads), lds, st, px, pd, part, g, splits);
      break;
  }
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

}  // namespace

bool dw_volume_supported(int64_t h, int64_t w) { return h >= 1 && w >= 1 && h * w <= kVolThreads; }

int dw_volume_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n, int64_t c, int64_t d,
                      int64_t h, int64_t w, int k, int dtype, bool flip, int seg, int depth_chunk, hipStream_t st) {
  VolGeom g{};
  size_t lds = 0;
  if (int status = volume_plan(n, c, d, h, w, k, dtype, seg, depth_chunk, false, &g, &lds)) return status;
#define MEDNEXT_VOL_STENCIL(T) \
  return flip ? volume_stencil_t<T, true>(x, weight, bias, y, g, k, lds, st) \
              : volume_stencil_t<T, false>(x, weight, bias, y, g, k, lds, st)
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: MEDNEXT_VOL_STENCIL(float);
    case MEDNEXT_DTYPE_F64: MEDNEXT_VOL_STENCIL(double);
    case MEDNEXT_DTYPE_F16: MEDNEXT_VOL_STENCIL(f16_t);
    default: MEDNEXT_VOL_STENCIL(bf16_t);
  }
#undef MEDNEXT_VOL_STENCIL
}

int dw_volume_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int seg,
                           int depth_chunk) {
  VolGeom g{};
  size_t lds = 0;
  if (volume_plan(n, c, d, h, w, k, dtype, seg, depth_chunk, true, &g, &lds) != MEDNEXT_STATUS_OK) return 0;
  const int64_t splits = n * g.nDc;
  return splits < (int64_t(1) << 31) ? static_cast<int>(splits) : 0;
}

int dw_volume_wgrad(const void* x, const void* dy, void* partial, int64_t n, int64_t c, int64_t d, int64_t h,
                    int64_t w, int k, int dtype, int seg, int depth_chunk, hipStream_t st) {
  VolGeom g{};
  size_t lds = 0;
  if (int status = volume_plan(n, c, d, h, w, k, dtype, seg, depth_chunk, true, &g, &lds)) return status;
  const int64_t splits = n * g.nDc;
  MEDNEXT_CHECK_ARG(splits < (int64_t(1) << 31), "too many partials");
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: return volume_wgrad_t<float>(x, dy, partial, g, k, static_cast<int>(splits), lds, st);
    case MEDNEXT_DTYPE_F64: return volume_wgrad_t<double>(x, dy, partial, g, k, static_cast<int>(splits), lds, st);
    case MEDNEXT_DTYPE_F16: return volume_wgrad_t<f16_t>(x, dy, partial, g, k, static_cast<int>(splits), lds, st);
    default: return volume_wgrad_t<bf16_t>(x, dy, partial, g, k, static_cast<int>(splits), lds, st);
  }
}

}  // namespace mednext
