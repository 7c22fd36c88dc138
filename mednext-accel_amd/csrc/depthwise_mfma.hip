// bf16 depthwise Conv3d on CDNA4 matrix cores: forward, input gradient (same
// stencil with flipped taps) and weight gradient (+ fused bias-grad sums).
//
// Stencil formulation. For one output tile of 16 columns (w0..w0+15) x 16 rows
// of a plane and one tap pair (kd, kh), the k taps along W form a banded
// Toeplitz matrix, so the 1-D correlation along W is one GEMM:
//   C[i][n] += sum_kk A[i][kk] * B[kk][n]
//   A[i][kk] = tap(kd, kh, kw = kk - 8 - i + p)   (zero outside 0 <= kw < k)
//   B[kk][n] = x[d][h0 + n + kh - p][w0 - 8 + kk],  kk in [0, 32)
// i.e. one v_mfma_f32_16x16x32_bf16 (fp32 accumulate). The K window starts at
// w0 - 8 so both the global->LDS fill and the B-operand LDS reads are 16-byte
// aligned. B for tap row kh is the same LDS tile read kh rows lower. Along D
// the kernel scatters: each input plane is read once and feeds k output planes held in
// rotating accumulators (an output plane is complete k-1 planes after its
// first contribution).
//
// Memory pipeline. Input planes are double-buffered in LDS; the global loads
// for plane i + PD are issued (into one of PD register sets) before plane i's
// MFMAs, so PD planes per workgroup are in flight while the matrix cores run.
// The compiler waits only for the set being stored. PD divides k so every
// register-set index is static under the k-fold unroll.
//
// Buffer helpers and the MFMA lane layout: cdna4.h.
#include "cdna4.h"
#include "common.h"
#include "depthwise_mfma.h"

namespace mednext {
namespace {

constexpr int kThreads = 256;
constexpr int kRT = 2;  // 16-row tiles per workgroup plane (32 rows)

struct MGeom {
  int C, D, H, W;
  int TD;  // output planes per workgroup
  int nDc, nHt, nWt;
};

struct BlockPos {
  int64_t nc;
  int c, n, dc, ht, wt;
};

__device__ inline BlockPos block_pos(const MGeom& g) {
  BlockPos b;
  int64_t bid = blockIdx.x;
  b.wt = static_cast<int>(bid % g.nWt);
  bid /= g.nWt;
  b.ht = static_cast<int>(bid % g.nHt);
  bid /= g.nHt;
  b.dc = static_cast<int>(bid % g.nDc);
  bid /= g.nDc;
  b.nc = bid;
  b.c = static_cast<int>(bid % g.C);
  b.n = static_cast<int>(bid / g.C);
  return b;
}

__device__ inline uint4 lds_read16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// ------------------------------------------------------------------ stencil

template <int K, bool FLIP, bool BIAS, int CT, int PD>
__global__ __launch_bounds__(kThreads) void dw_mfma_stencil_kernel(const bf16_t* __restrict__ x,
                                                                   const bf16_t* __restrict__ wt,
                                                                   const bf16_t* __restrict__ bias,
                                                                   bf16_t* __restrict__ y,
                                                                   MGeom g) {
  constexpr int P = K / 2;
  constexpr int K3 = K * K * K;
  constexpr int TH = 16 * kRT, TW = 16 * CT;
  constexpr int LR = TH + 2 * P;  // LDS rows: h = th0 - P + r
  constexpr int LC = TW + 16;     // LDS cols: w = tw0 - 8 + col
  constexpr int CPR = LC / 8;     // 16-byte chunks per LDS row
  constexpr int NCHUNK = LR * CPR;
  constexpr int NCH = (NCHUNK + kThreads - 1) / kThreads;
  constexpr int TPW = kRT * CT / 4;  // tiles per wave
  static_assert(K % PD == 0, "prefetch depth must divide k");
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint16_t* lds = reinterpret_cast<uint16_t*>(smem_raw);

  const BlockPos bp = block_pos(g);
  const int th0 = bp.ht * TH, tw0 = bp.wt * TW, d0 = bp.dc * g.TD;
  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const uint16_t* __restrict__ xnc = reinterpret_cast<const uint16_t*>(x) + bp.nc * g.D * plane;
  uint16_t* __restrict__ ync = reinterpret_cast<uint16_t*>(y) + bp.nc * g.D * plane;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n16 = lane & 15;
  const int q = lane >> 4;

  // A operands: Toeplitz tap matrices, one per (kd, kh).
  bf16x8_t amat[K][K];
  {
    const uint16_t* __restrict__ wraw =
        reinterpret_cast<const uint16_t*>(wt) + static_cast<int64_t>(bp.c) * K3;
#pragma unroll
    for (int kd = 0; kd < K; ++kd)
#pragma unroll
      for (int kh = 0; kh < K; ++kh)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int kw = 8 * q + j - 8 - n16 + P;
          uint16_t bits = 0;
          if (kw >= 0 && kw < K) {
            const int t = (kd * K + kh) * K + kw;
            bits = wraw[FLIP ? K3 - 1 - t : t];
          }
          amat[kd][kh][j] = __builtin_bit_cast(__bf16, bits);
        }
  }
  float b0 = 0.f;
  if constexpr (BIAS) b0 = bf16_to_f32(reinterpret_cast<const uint16_t*>(bias)[bp.c]);
  const f32x4_t acc_init = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Per-thread chunk coordinates of the fill (the same for every plane).
  // Threads without a chunk write a dummy LDS slot past the two buffers.
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(xnc, static_cast<uint32_t>(g.D * plane * 2));
  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(ync, static_cast<uint32_t>(g.D * plane * 2));
  int ch_off[NCH];  // byte offset inside a plane, or -1 outside the plane
  int ch_lds[NCH];  // LDS element offset
#pragma unroll
  for (int u = 0; u < NCH; ++u) {
    const int e = threadIdx.x + u * kThreads;
    ch_off[u] = -1;
    ch_lds[u] = 2 * LR * LC;
    if (e < NCHUNK) {
      const int r = e / CPR;
      const int ch = e - r * CPR;
      const int h = th0 - P + r;
      const int w = tw0 - 8 + 8 * ch;
      ch_lds[u] = r * LC + 8 * ch;
      if (h >= 0 && h < g.H && w >= 0 && w < g.W) ch_off[u] = 2 * (h * g.W + w);
    }
  }
  const int nplanes = g.TD + K - 1;
  // Input plane j of this workgroup (absolute d0 - P + j); planes outside the
  // volume or past this workgroup's range read as zeros without touching memory.
  auto load_plane = [&](int j, uint4* pre) {
    const int di = d0 - P + j;
    const bool plane_ok = j < nplanes && di >= 0 && di < g.D;
    const uint32_t pbase = static_cast<uint32_t>(plane_ok ? di : 0) * static_cast<uint32_t>(plane * 2);
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      const uint32_t off = (plane_ok && ch_off[u] >= 0) ? pbase + static_cast<uint32_t>(ch_off[u]) : kOob;
      pre[u] = buf_load16(xr, off);  // halo rows/planes are re-read: keep them cacheable
    }
  };
  auto store_plane = [&](uint16_t* buf, const uint4* pre) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) *reinterpret_cast<uint4*>(buf + ch_lds[u]) = pre[u];
  };

  f32x4_t acc[K][TPW];
#pragma unroll
  for (int s = 0; s < K; ++s)
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[s][t] = acc_init;

  uint4 pre[PD][NCH];
  load_plane(0, pre[0]);
  store_plane(lds, pre[0]);
#pragma unroll
  for (int j = 1; j <= PD; ++j) load_plane(j, pre[(j - 1) % PD]);
  __syncthreads();

  for (int q0 = 0; q0 < nplanes; q0 += K) {
#pragma unroll
    for (int s = 0; s < K; ++s) {
      const int i = q0 + s;
      if (i >= nplanes) break;
      load_plane(i + PD, pre[(s + PD - 1) % PD]);
      const uint16_t* buf = lds + (i & 1) * LR * LC;
      const int o = i - (K - 1);  // output plane completed by this input plane
      const int cs = (s + 1) % K;
      const bool write_o = o >= 0 && o < g.TD && d0 + o < g.D;
      const uint32_t obase = static_cast<uint32_t>(write_o ? d0 + o : 0) * static_cast<uint32_t>(plane * 2);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int tile = wave + 4 * t;
        const int ty = tile / CT;
        const int tx = tile % CT;
        const uint16_t* bp0 = buf + (16 * ty + n16) * LC + 16 * tx + 8 * q;
#pragma unroll
        for (int kh = 0; kh < K; ++kh) {
          const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, lds_read16(bp0 + kh * LC));
#pragma unroll
          for (int kd = 0; kd < K; ++kd) {
            const int slot = ((s - kd) % K + K) % K;
            acc[slot][t] =
                __builtin_amdgcn_mfma_f32_16x16x32_bf16(amat[kd][kh], bm, acc[slot][t], 0, 0, 0);
          }
        }
        {
          const int h = th0 + 16 * ty + n16;
          const int w = tw0 + 16 * tx + 4 * q;
          const bool ok = write_o && h < g.H && w < g.W;
          const uint32_t off = ok ? obase + static_cast<uint32_t>(2 * (h * g.W + w)) : kOob;
          const f32x4_t a = acc[cs][t];
          const bf16x4_t packed = {static_cast<__bf16>(a[0] + b0), static_cast<__bf16>(a[1] + b0),
                                   static_cast<__bf16>(a[2] + b0), static_cast<__bf16>(a[3] + b0)};
          const u32x2_t words = __builtin_bit_cast(u32x2_t, packed);
          buf_store8(yr, off, words[0], words[1]);
        }
        acc[cs][t] = acc_init;
      }
      store_plane(lds + ((i + 1) & 1) * LR * LC, pre[s % PD]);
      __syncthreads();
    }
  }
}


// ------------------------------------------------------------ weight gradient
//
// dW[kd][kh][kw] = sum_{o,h,w} x[o+kd-p][h+kh-p][w+kw-p] * dy[o][h][w] on matrix
// cores. For one input plane i, one row h and 32 output columns w0..w0+31:
//   C[m][n] += sum_kk A[m][kk] * B[kk][n]
//   m = kh*k + kw (taps of one plane; 16 rows per MFMA, two MFMAs for k = 5)
//   n = kd (the k grad_output planes o = i - kd; columns n >= k are unused)
//   A[m][kk] = x[i][h + kh - p][w0 + kk + kw - p]
//   B[kk][n] = dy[i - n][h][w0 + kk]
// so C[m][n] accumulates the partial sum of tap (kd = n, kh, kw) over the
// whole workgroup in one 16x16 fp32 tile per wave. Row m = k^2 of A is all
// ones, so C[k^2][0] accumulates the bias gradient (sum of dy) for free.
// A needs a per-lane column shift (kw - p): LDS holds k copies of the x tile,
// copy s shifted by s - p columns, so every A operand is one aligned 16-byte
// read; row and copy strides are padded so the 8 lanes of each 16-byte LDS
// phase hit distinct banks. grad_output planes live in a (k+1)-slot LDS ring,
// so the slot being refilled is never one the current plane reads. A
// workgroup covers 16*RT full rows (16*CT >= W columns): column halos fall
// outside the row and cost no memory traffic. Each wave owns a fixed band of
// rows. Loads for plane i + PD are in flight (non-temporal) while plane i's
// MFMAs run. Per-workgroup partials go to a fp32 workspace reduced in fixed
// order afterwards.
template <int K, int CT, int RT>
struct WgradLayout {
  static constexpr int P = K / 2;
  static constexpr int TH = 16 * RT, TW = 16 * CT;
  static constexpr int LR = TH + 2 * P;         // x rows: h = th0 - P + r
  static constexpr int XROW = TW + 8;           // elements; 4 dwords mod 32 dwords
  static constexpr int XCOPY_RAW = LR * XROW;   // elements per shifted copy
  // copy stride == 12 dwords (24 elements) mod 64 elements
  static constexpr int XCOPY = XCOPY_RAW + ((24 - XCOPY_RAW % 64) % 64 + 64) % 64;
  static constexpr int XBUF = K * XCOPY;        // elements per plane buffer
  static constexpr int DSLOT = TH * TW + 8;     // dy slot stride (elements)
  static constexpr int RING = K + 1;
  static constexpr int XDUMMY = 2 * XBUF;       // K x 8 elements for chunkless threads
  static constexpr int RING_OFF = XDUMMY + 8 * K;
  static constexpr int DDUMMY = RING_OFF + RING * DSLOT;
  static constexpr size_t bytes = static_cast<size_t>(DDUMMY + 8) * 2;
};

template <int K, int CT, int RT, int PD>
__global__ __launch_bounds__(kThreads) void dw_mfma_wgrad_kernel(const bf16_t* __restrict__ x,
                                                                 const bf16_t* __restrict__ dy,
                                                                 float* __restrict__ partial,
                                                                 MGeom g, int splits) {
  using L = WgradLayout<K, CT, RT>;
  constexpr int P = K / 2;
  constexpr int K2 = K * K;
  constexpr int K3 = K2 * K;
  constexpr int MB = (K2 + 1 + 15) / 16;  // taps plus the all-ones row
  constexpr int TH = L::TH, TW = L::TW, LR = L::LR;
  constexpr int XCPR = TW / 8;  // 8-element chunks per row
  constexpr int XCHUNKS = LR * XCPR;
  constexpr int NXC = (XCHUNKS + kThreads - 1) / kThreads;
  constexpr int DCHUNKS = TH * XCPR;
  constexpr int NDC = (DCHUNKS + kThreads - 1) / kThreads;
  constexpr int UPR = TW / 32;  // 32-column MFMA units per row
  constexpr int ROWS_PER_WAVE = TH / 4;
  constexpr int RING = L::RING;
  static_assert(P <= 2, "the fill builds column shifts of at most 2");
  extern __shared__ __align__(16) unsigned char smem_raw[];

  const BlockPos bp = block_pos(g);
  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem_raw);
  uint16_t* const ring = lds + L::RING_OFF;  // [RING][DSLOT]
  const int th0 = bp.ht * TH, tw0 = bp.wt * TW, d0 = bp.dc * g.TD;
  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const uint16_t* __restrict__ xnc = reinterpret_cast<const uint16_t*>(x) + bp.nc * g.D * plane;
  const uint16_t* __restrict__ dync = reinterpret_cast<const uint16_t*>(dy) + bp.nc * g.D * plane;
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(xnc, static_cast<uint32_t>(g.D * plane * 2));
  const __amdgpu_buffer_rsrc_t dr = slab_rsrc(dync, static_cast<uint32_t>(g.D * plane * 2));
  const int nplanes = g.TD + K - 1;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n16 = lane & 15;
  const int q = lane >> 4;

  // Fill coordinates, the same for every plane. A chunk is x[w .. w+7] of one
  // row (w = tw0 + 8*ch); the shifted copies also need the dwords just before
  // (x[w-2], x[w-1]) and after (x[w+8], x[w+9]). Offsets are bytes inside a
  // plane (-1: outside it). Threads without a chunk write dummy LDS slots.
  int x_main[NXC], x_prev[NXC], x_next[NXC], x_lds[NXC], x_step[NXC];
#pragma unroll
  for (int u = 0; u < NXC; ++u) {
    const int e = threadIdx.x + u * kThreads;
    x_main[u] = x_prev[u] = x_next[u] = -1;
    x_lds[u] = L::XDUMMY;
    x_step[u] = 8;  // dummy: copies at consecutive 16-byte slots
    if (e < XCHUNKS) {
      const int r = e / XCPR;
      const int ch = e - r * XCPR;
      const int h = th0 - P + r;
      const int w = tw0 + 8 * ch;
      x_lds[u] = r * L::XROW + 8 * ch;
      x_step[u] = L::XCOPY;
      if (h >= 0 && h < g.H) {
        const int pos = h * g.W + w;
        if (w < g.W) x_main[u] = 2 * pos;
        if (w >= 8 && w - 8 < g.W) x_prev[u] = 2 * (pos - 2);
        if (w + 8 < g.W) x_next[u] = 2 * (pos + 8);
      }
    }
  }
  int d_off[NDC], d_lds[NDC];
#pragma unroll
  for (int u = 0; u < NDC; ++u) {
    const int e = threadIdx.x + u * kThreads;
    d_off[u] = -1;
    d_lds[u] = -1;  // -1: dummy slot
    if (e < DCHUNKS) {
      const int r = e / XCPR;
      const int ch = e - r * XCPR;
      const int h = th0 + r;
      const int w = tw0 + 8 * ch;
      d_lds[u] = r * TW + 8 * ch;
      if (h < g.H && w < g.W) d_off[u] = 2 * (h * g.W + w);
    }
  }

  struct Pre {
    uint4 xv[NXC];
    uint32_t pw[NXC];
    uint32_t nw[NXC];
    uint4 dv[NDC];
  };
  // Plane j of this workgroup: x plane d0 - P + j and grad_output plane d0 + j.
  auto load = [&](int j, Pre& p) {
    const int di = d0 - P + j;
    const bool xok = j < nplanes && di >= 0 && di < g.D;
    const uint32_t xbase = static_cast<uint32_t>(xok ? di : 0) * static_cast<uint32_t>(plane * 2);
#pragma unroll
    for (int u = 0; u < NXC; ++u) {
      p.xv[u] = buf_load16(xr, xok && x_main[u] >= 0 ? xbase + x_main[u] : kOob);
      p.pw[u] = buf_load4(xr, xok && x_prev[u] >= 0 ? xbase + x_prev[u] : kOob);
      p.nw[u] = buf_load4(xr, xok && x_next[u] >= 0 ? xbase + x_next[u] : kOob);
    }
    const bool dok = j < g.TD && d0 + j < g.D;
    const uint32_t dbase = static_cast<uint32_t>(dok ? d0 + j : 0) * static_cast<uint32_t>(plane * 2);
#pragma unroll
    for (int u = 0; u < NDC; ++u) {
      p.dv[u] = buf_load16_nt(dr, dok && d_off[u] >= 0 ? dbase + d_off[u] : kOob);
    }
  };
  auto store = [&](int i, const Pre& p) {
    uint16_t* const buf = lds + (i & 1) * L::XBUF;
#pragma unroll
    for (int u = 0; u < NXC; ++u) {
      // Words of x[w-2 .. w+9]: e[0] = (x[w-2], x[w-1]), e[1..4] = the chunk,
      // e[5] = (x[w+8], x[w+9]). Copy s (shift s - P) starts at x[w + s - P].
      const uint32_t e[6] = {p.pw[u], p.xv[u].x, p.xv[u].y, p.xv[u].z, p.xv[u].w, p.nw[u]};
      uint16_t* const dst = (x_lds[u] == L::XDUMMY ? lds : buf) + x_lds[u];
#pragma unroll
      for (int cs = 0; cs < K; ++cs) {
        const int sh = cs - P;  // -2..2 elements
        uint4 v;
        if (sh % 2 == 0) {
          const int b = 1 + sh / 2;
          v = make_uint4(e[b], e[b + 1], e[b + 2], e[b + 3]);
        } else {
          // Odd shift: word j = (x[w+sh+2j], x[w+sh+2j+1]) is the high half
          // of e[b+j] and the low half of e[b+j+1].
          const int b = sh < 0 ? 0 : 1;
          v = make_uint4(__builtin_amdgcn_alignbit(e[b + 1], e[b], 16),
                         __builtin_amdgcn_alignbit(e[b + 2], e[b + 1], 16),
                         __builtin_amdgcn_alignbit(e[b + 3], e[b + 2], 16),
                         __builtin_amdgcn_alignbit(e[b + 4], e[b + 3], 16));
        }
        *reinterpret_cast<uint4*>(dst + cs * x_step[u]) = v;
      }
    }
    uint16_t* const slot = ring + (i % RING) * L::DSLOT;
#pragma unroll
    for (int u = 0; u < NDC; ++u) {
      uint16_t* const dst = d_lds[u] < 0 ? lds + L::DDUMMY : slot + d_lds[u];
      *reinterpret_cast<uint4*>(dst) = p.dv[u];
    }
  };

  // Zero the grad_output ring (planes before the first and past the last are zero).
  for (int e = threadIdx.x; e < RING * L::DSLOT / 8; e += kThreads) {
    reinterpret_cast<uint4*>(ring)[e] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();

  // Per-lane operand geometry and the constant rows of A.
  int a_off[MB];
  bool a_ok[MB];
  uint4 av[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int m = 16 * mb + n16;
    a_ok[mb] = m < K2;
    const int kh = a_ok[mb] ? m / K : 0;
    const int kw = a_ok[mb] ? m - kh * K : 0;
    a_off[mb] = kw * L::XCOPY + (wave * ROWS_PER_WAVE + kh) * L::XROW + 8 * q;
    const uint32_t fill = m == K2 ? 0x3F803F80u : 0u;  // bf16 ones for the bias row
    av[mb] = make_uint4(fill, fill, fill, fill);
  }
  const bool b_ok = n16 < K;
  const int b_off = wave * ROWS_PER_WAVE * TW + 8 * q;
  uint4 bv = make_uint4(0u, 0u, 0u, 0u);

  Pre pre[PD];
  {
    Pre first;
    load(0, first);
    store(0, first);
  }
#pragma unroll
  for (int j = 1; j <= PD; ++j) load(j, pre[(j - 1) % PD]);
  __syncthreads();

  f32x4_t acc[UPR][MB];
#pragma unroll
  for (int u = 0; u < UPR; ++u)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[u][mb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  for (int i0 = 0; i0 < nplanes; i0 += PD) {
#pragma unroll
    for (int s = 0; s < PD; ++s) {
      const int i = i0 + s;
      if (i >= nplanes) break;
      load(i + PD, pre[(s + PD - 1) % PD]);
      const uint16_t* const xb = lds + (i & 1) * L::XBUF;
      // Lane n reads grad_output plane i - n; slots of planes < 0 hold zeros.
      const int o = i - n16;
      const uint16_t* const bslot = ring + ((o % RING + RING) % RING) * L::DSLOT + b_off;
#pragma unroll
      for (int rr = 0; rr < ROWS_PER_WAVE; ++rr) {
        // Operands of the row's UPR units first, then UPR independent MFMA
        // chains (one accumulator set per unit).
        uint4 bvs[UPR];
        uint4 avs[UPR][MB];
#pragma unroll
        for (int u = 0; u < UPR; ++u) {
          bvs[u] = bv;
          if (b_ok) bvs[u] = lds_read16(bslot + rr * TW + 32 * u);
#pragma unroll
          for (int mb = 0; mb < MB; ++mb) {
            avs[u][mb] = av[mb];
            if (a_ok[mb]) avs[u][mb] = lds_read16(xb + a_off[mb] + rr * L::XROW + 32 * u);
          }
        }
#pragma unroll
        for (int u = 0; u < UPR; ++u)
#pragma unroll
          for (int mb = 0; mb < MB; ++mb)
            acc[u][mb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf16x8_t, avs[u][mb]), __builtin_bit_cast(bf16x8_t, bvs[u]),
                acc[u][mb], 0, 0, 0);
      }
      store(i + 1, pre[s % PD]);
      __syncthreads();
    }
  }

  // Reduce the four waves' tiles in a fixed order. Tap t = kd*k^2 + m sits at
  // C[m][kd]; the bias gradient at C[k^2][0].
  float* red = reinterpret_cast<float*>(smem_raw);  // reuse LDS: [4][MB][256]
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    f32x4_t sum = acc[0][mb];
#pragma unroll
    for (int u = 1; u < UPR; ++u) sum += acc[u][mb];
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * MB + mb) * 256 + (4 * q + r) * 16 + n16] = sum[r];
  }
  __syncthreads();
  const int64_t split =
      ((static_cast<int64_t>(bp.n) * g.nDc + bp.dc) * g.nHt + bp.ht) * g.nWt + bp.wt;
  for (int t = threadIdx.x; t < K3 + 1; t += kThreads) {
    int m, kd;
    if (t < K3) {
      kd = t / K2;
      m = t - kd * K2;
    } else {
      kd = 0;
      m = K2;
    }
    const int mb = m >> 4;
    const int idx = (m & 15) * 16 + kd;
    const float v = red[(0 * MB + mb) * 256 + idx] + red[(1 * MB + mb) * 256 + idx] +
                    red[(2 * MB + mb) * 256 + idx] + red[(3 * MB + mb) * 256 + idx];
    partial[(static_cast<int64_t>(bp.c) * (K3 + 1) + t) * splits + split] = v;
  }
}

// ------------------------------------------------------------------ host side

int make_geom(int64_t c, int64_t d, int64_t h, int64_t w, int tile_cols, int depth_chunk,
              MGeom* g) {
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  MEDNEXT_CHECK_ARG(h * w < (int64_t(1) << 31), "plane must have < 2^31 elements");
  g->C = static_cast<int>(c);
  g->D = static_cast<int>(d);
  g->H = static_cast<int>(h);
  g->W = static_cast<int>(w);
  g->TD = static_cast<int>(depth_chunk < d ? depth_chunk : d);
  g->nDc = static_cast<int>(cdiv(d, g->TD));
  g->nHt = static_cast<int>(cdiv(h, 16 * kRT));
  g->nWt = static_cast<int>(cdiv(w, tile_cols));
  return MEDNEXT_STATUS_OK;
}

template <int K, bool FLIP, int CT, int PD>
int launch_stencil(const void* x, const void* wt, const void* bias, void* y, const MGeom& g,
                   int64_t blocks, hipStream_t st) {
  constexpr int P = K / 2;
  // two plane buffers + one dummy 16-byte slot for threads without a fill chunk
  constexpr size_t lds = (static_cast<size_t>(2) * (16 * kRT + 2 * P) * (16 * CT + 16) + 8) * 2;
  auto px = static_cast<const bf16_t*>(x);
  auto pw = static_cast<const bf16_t*>(wt);
  auto pb = static_cast<const bf16_t*>(bias);
  auto py = static_cast<bf16_t*>(y);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
  if (bias)
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, true, CT, PD>), grid, block, lds, st, px,
                       pw, pb, py, g);
  else
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, false, CT, PD>), grid, block, lds, st, px,
                       pw, pb, py, g);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <int K, bool FLIP>
int launch_stencil_ct(const void* x, const void* wt, const void* bias, void* y, const MGeom& g,
                      int tile_cols, int64_t blocks, hipStream_t st) {
  constexpr int PD = K == 3 ? 3 : 1;
  switch (tile_cols) {
    case 32: return launch_stencil<K, FLIP, 2, PD>(x, wt, bias, y, g, blocks, st);
    case 64: return launch_stencil<K, FLIP, 4, PD>(x, wt, bias, y, g, blocks, st);
    default: return launch_stencil<K, FLIP, 8, PD>(x, wt, bias, y, g, blocks, st);
  }
}


template <int K, int CT, int RT>
size_t wgrad_lds_bytes() {
  constexpr int MB = (K * K + 1 + 15) / 16;
  constexpr size_t red = static_cast<size_t>(4 * MB * 256) * 4;
  return WgradLayout<K, CT, RT>::bytes > red ? WgradLayout<K, CT, RT>::bytes : red;
}

template <int K, int CT>
int launch_wgrad(const void* x, const void* dy, float* partial, const MGeom& g, int64_t blocks,
                 int splits, hipStream_t st) {
  constexpr int PD = 2;
  constexpr int RT = 1;
  const size_t lds = wgrad_lds_bytes<K, CT, RT>();
  hipLaunchKernelGGL((dw_mfma_wgrad_kernel<K, CT, RT, PD>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kThreads), lds, st, static_cast<const bf16_t*>(x),
                     static_cast<const bf16_t*>(dy), partial, g, splits);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

// Weight-gradient workgroups cover 16 full rows (16 * RT with RT = 1).
constexpr int kWgradRows = 16;

int plan_wgrad(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int tile_cols,
               int depth_chunk, MGeom* g, int64_t* blocks, int* splits) {
  MEDNEXT_CHECK_ARG(dw_mfma_supported(d, h, w, k) && w % 32 == 0,
                    "MFMA wgrad needs k in {3,5}, W % 32 == 0, H >= 32 and a slab < 2 GiB");
  MEDNEXT_CHECK_ARG(tile_cols == 32 || tile_cols == 64 || tile_cols == 128,
                    "MFMA wgrad tile_w must be 32, 64 or 128");
  int st = make_geom(c, d, h, w, tile_cols, depth_chunk, g);
  if (st != MEDNEXT_STATUS_OK) return st;
  g->nHt = static_cast<int>(cdiv(h, kWgradRows));
  *blocks = n * c * g->nDc * g->nHt * g->nWt;
  MEDNEXT_CHECK_ARG(*blocks < (int64_t(1) << 31), "grid too large");
  *splits = static_cast<int>(n * g->nDc * g->nHt * g->nWt);
  return MEDNEXT_STATUS_OK;
}

}  // namespace

bool dw_mfma_supported(int64_t d, int64_t h, int64_t w, int k) {
  // Buffer offsets are 32-bit: one (n, c) slab must stay below 2 GiB.
  return (k == 3 || k == 5) && w % 8 == 0 && w >= 32 && h >= 32 && d >= 1 &&
         d * h * w * 2 < (int64_t(1) << 31);
}

int dw_mfma_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n,
                    int64_t c, int64_t d, int64_t h, int64_t w, int k, bool flip, int tile_cols,
                    int depth_chunk, hipStream_t st) {
  MEDNEXT_CHECK_ARG(dw_mfma_supported(d, h, w, k),
                    "MFMA stencil needs k in {3,5}, W % 8 == 0, W >= 32, H >= 32 and a slab < 2 GiB");
  MEDNEXT_CHECK_ARG(tile_cols == 32 || tile_cols == 64 || tile_cols == 128,
                    "MFMA tile_w must be 32, 64 or 128");
  MGeom g{};
  int status = make_geom(c, d, h, w, tile_cols, depth_chunk, &g);
  if (status != MEDNEXT_STATUS_OK) return status;
  const int64_t blocks = n * c * g.nDc * g.nHt * g.nWt;
  MEDNEXT_CHECK_ARG(blocks < (int64_t(1) << 31), "grid too large");
  if (k == 3) {
    return flip ? launch_stencil_ct<3, true>(x, weight, bias, y, g, tile_cols, blocks, st)
                : launch_stencil_ct<3, false>(x, weight, bias, y, g, tile_cols, blocks, st);
  }
  return flip ? launch_stencil_ct<5, true>(x, weight, bias, y, g, tile_cols, blocks, st)
              : launch_stencil_ct<5, false>(x, weight, bias, y, g, tile_cols, blocks, st);
}


int dw_mfma_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k,
                         int tile_cols, int depth_chunk) {
  MGeom g{};
  int64_t blocks = 0;
  int splits = 0;
  if (plan_wgrad(n, c, d, h, w, k, tile_cols, depth_chunk, &g, &blocks, &splits) !=
      MEDNEXT_STATUS_OK)
    return 0;
  return splits;
}

int dw_mfma_wgrad(const void* x, const void* dy, float* partial, int64_t n, int64_t c, int64_t d,
                  int64_t h, int64_t w, int k, int tile_cols, int depth_chunk, hipStream_t st) {
  MGeom g{};
  int64_t blocks = 0;
  int splits = 0;
  int status = plan_wgrad(n, c, d, h, w, k, tile_cols, depth_chunk, &g, &blocks, &splits);
  if (status != MEDNEXT_STATUS_OK) return status;
  if (k == 3) {
    switch (tile_cols) {
      case 32: return launch_wgrad<3, 2>(x, dy, partial, g, blocks, splits, st);
      case 64: return launch_wgrad<3, 4>(x, dy, partial, g, blocks, splits, st);
      default: return launch_wgrad<3, 8>(x, dy, partial, g, blocks, splits, st);
    }
  }
  switch (tile_cols) {
    case 32: return launch_wgrad<5, 2>(x, dy, partial, g, blocks, splits, st);
    case 64: return launch_wgrad<5, 4>(x, dy, partial, g, blocks, splits, st);
    default: return launch_wgrad<5, 8>(x, dy, partial, g, blocks, splits, st);
  }
}

}  // namespace mednext
