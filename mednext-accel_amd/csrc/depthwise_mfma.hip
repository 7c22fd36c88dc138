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
// The compiler waits only for the set being stored. The plane loop is
// unrolled by lcm(k, PD), so every register-set and accumulator index is
// static. For k = 3 finished output planes leave through an LDS staging tile
// as whole rows (16-byte stores).
//
// Block-Toeplitz form (k = 5). The 1-D form spends k^2 = 25 MFMAs per tile
// and input plane, 5 of every 32 products useful. For k = 5 the 16x16 tile is
// instead 16 blocks of 4x4 outputs (n = block, i = 4 * row + col inside it)
// and the K window is a 4-row x 8-column piece of the block's 8x8 input
// window, so two MFMAs (input rows 0-3 and 4-7 of the window) cover all 25
// taps of one kd:
//   A_{kd,h}[i][8 r + c] = tap(kd, kh = 4 h + r - i / 4, kw = c - i % 4)
//   B_h[8 r + c][n]      = x[d][h0(n) + 4 h + r - p][w0(n) + c - p]
// 10 MFMAs per tile and input plane (39% of the products useful), and ten
// instead of 25 tap matrices in registers. The B rows of one lane start two
// elements before a 4-aligned column, so they are read as four dwords; the
// LDS row pitch is padded to an odd multiple of four dwords so the 16 blocks
// of a lane group fall on distinct banks.
//
// Stride-2 modes. The MedNeXt down block's stride-2 depthwise conv (padding
// k/2) and its input gradient are this stencil in disguise:
//   gather  small[o] = sum_t w[t] big[2o + t - p] = stencil(big)[2o]
//   scatter big[i]   = sum_{2o + t - p = i} w[t] small[o]
//                    = flipped-tap stencil over up(small), up(small)[2o] =
//                      small[o] and zero at odd indices.
// kS2Sub runs the stencil over the big tensor and stores only the even output
// positions, into the small tensor, skipping the MFMAs of odd output planes;
// kS2Up fills the LDS planes from the small tensor, expanded with zeros, and
// skips the MFMAs of the all-zero odd input planes. The weight gradient's
// kS2 form (dW[t] = sum_o big[2o + t - p] small[o]) is the weight-gradient
// kernel below with dy = up(small).
//
// Buffer helpers and the MFMA lane layout: cdna4.h.
#include <algorithm>

#include "cdna4.h"
#include "common.h"
#include "depthwise_mfma.h"

namespace mednext {
namespace {

constexpr int kThreads = 256;
constexpr int kRT = 2;  // 16-row tiles per workgroup plane (32 rows)

constexpr bool stencil_stages_output(int k) { return k == 3; }
constexpr int kS2None = 0, kS2Sub = 1, kS2Up = 2;  // stencil stride-2 modes
constexpr bool stencil_blocks(int k) { return k == 5; }
// LDS row pitch (elements) of the plane buffers: [tw0 - 8, tw0 + TW + 8), plus
// 8 elements of padding in the block-Toeplitz form.
constexpr int stencil_pitch(int k, int ct) { return 16 * ct + (stencil_blocks(k) ? 24 : 16); }
constexpr int gcd_int(int a, int b) { return b == 0 ? a : gcd_int(b, a % b); }
constexpr int lcm_int(int a, int b) { return a / gcd_int(a, b) * b; }

struct MGeom {
  int C, D, H, W;  // the stencil's (big) grid
  int TD;  // output planes per workgroup
  int nDc, nHt, nWt;
  int Ds, Hs, Ws;  // stride-2 modes: the small tensor
};

struct BlockPos {
  int64_t nc;
  int c, n, dc, ht, wt;
};

__device__ inline BlockPos block_pos(const MGeom& g) {
  BlockPos b;
  int64_t bid = xcd_swizzle(blockIdx.x, gridDim.x);
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

// ACC (input gradient): y = stencil + acc, acc a tensor shaped
// like y (the gradient that reaches the same input through the block's
// residual), added to the bf16-rounded stencil value in fp32 and rounded
// again, exactly as a separate bf16 add would.
// EW (stride-2 modes on big tensors of odd width, the up block's 2s - 1):
// the big tensor's rows are not 16-byte aligned, so kS2Sub reads it with
// run8_load / run8_pack and kS2Up writes it with 2-byte stores.
template <int K, bool FLIP, bool BIAS, int CT, int PD, bool ACC = false, int S2 = kS2None, bool EW = false>
__global__ __launch_bounds__(kThreads) void dw_mfma_stencil_kernel(const bf16_t* __restrict__ x,
                                                                   const bf16_t* __restrict__ wt,
                                                                   const bf16_t* __restrict__ bias,
                                                                   bf16_t* __restrict__ y,
                                                                   MGeom g,
                                                                   const bf16_t* __restrict__ acc_in = nullptr) {
  constexpr int P = K / 2;
  constexpr int K3 = K * K * K;
  constexpr int TH = 16 * kRT, TW = 16 * CT;
  constexpr bool BLK = stencil_blocks(K);
  constexpr int LR = TH + 2 * P;              // LDS rows: h = th0 - P + r
  constexpr int LC = stencil_pitch(K, CT);    // LDS cols: w = tw0 - 8 + col
  constexpr int CPR = (TW + 16) / 8;          // 16-byte chunks per LDS row
  constexpr int NCHUNK = LR * CPR;
  constexpr int NCH = (NCHUNK + kThreads - 1) / kThreads;
  constexpr int TPW = kRT * CT / 4;  // tiles per wave
  // k = 3: finished output planes are staged through LDS and written as whole
  // rows, 16 bytes per lane (an MFMA tile row holds only 4 consecutive
  // outputs per lane, i.e. 16 rows x 32-byte pieces per store instruction).
  // k = 5 keeps the direct 8-byte stores: its LDS and register footprint
  // already bound occupancy, and measured faster that way.
  constexpr bool STAGE = stencil_stages_output(K);
  static_assert(!(BLK && STAGE), "the block-Toeplitz form stores its outputs directly");
  static_assert(S2 == kS2None || !ACC, "stride-2 modes take no accumulation input");
  static_assert(!EW || S2 != kS2None, "element-exact rows are for the stride-2 modes");
  constexpr int OC = TW + 8;           // output staging row pitch (elements)
  constexpr int OBUF = TH * OC;
  constexpr int OCH = TH * (TW / 8);   // 16-byte output chunks per plane
  constexpr int NOC = (OCH + kThreads - 1) / kThreads;
  // The plane loop is unrolled by U = lcm(K, PD) so that both the rotating
  // accumulator slot (plane mod K) and the prefetch register set (plane mod
  // PD) are compile-time indices.
  constexpr int U = lcm_int(K, PD);
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint16_t* lds = reinterpret_cast<uint16_t*>(smem_raw);

  const BlockPos bp = block_pos(g);
  const int th0 = bp.ht * TH, tw0 = bp.wt * TW, d0 = bp.dc * g.TD;
  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const int64_t splane = static_cast<int64_t>(g.Hs) * g.Ws;  // stride-2 modes
  const int64_t in_slab = S2 == kS2Up ? g.Ds * splane : g.D * plane;
  const int64_t out_slab = S2 == kS2Sub ? g.Ds * splane : g.D * plane;
  const uint16_t* __restrict__ xnc = reinterpret_cast<const uint16_t*>(x) + bp.nc * in_slab;
  uint16_t* __restrict__ ync = reinterpret_cast<uint16_t*>(y) + bp.nc * out_slab;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n16 = lane & 15;
  const int q = lane >> 4;

  // A operands: Toeplitz tap matrices, one per (kd, kh); block-Toeplitz, one
  // per (kd, window half).
  constexpr int NA = BLK ? 2 : K;
  bf16x8_t amat[K][NA];
  {
    const uint16_t* __restrict__ wraw =
        reinterpret_cast<const uint16_t*>(wt) + static_cast<int64_t>(bp.c) * K3;
#pragma unroll
    for (int kd = 0; kd < K; ++kd)
#pragma unroll
      for (int a = 0; a < NA; ++a)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          // 1-D: row i = n16 is output column i, kk = 8 q + j the window column.
          // Block: i = n16 is output (n16 / 4, n16 % 4) of the block, kk = (q, j).
          const int kh = BLK ? 4 * a + q - (n16 >> 2) : a;
          const int kw = BLK ? j - (n16 & 3) : 8 * q + j - 8 - n16 + P;
          uint16_t bits = 0;
          if (kh >= 0 && kh < K && kw >= 0 && kw < K) {
            const int t = (kd * K + kh) * K + kw;
            bits = wraw[FLIP ? K3 - 1 - t : t];
          }
          amat[kd][a][j] = __builtin_bit_cast(__bf16, bits);
        }
  }
  float b0 = 0.f;
  if constexpr (BIAS) b0 = bf16_to_f32(reinterpret_cast<const uint16_t*>(bias)[bp.c]);
  const f32x4_t acc_init = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Per-thread chunk coordinates of the fill (the same for every plane).
  // Threads without a chunk (ch_lds -1) store nothing: their stores are
  // masked off (a shared sink address would serialise every such lane of an
  // instruction on one LDS bank).
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(xnc, static_cast<uint32_t>(in_slab * 2));
  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(ync, static_cast<uint32_t>(out_slab * 2));
  const __amdgpu_buffer_rsrc_t ar =
      slab_rsrc(ACC ? reinterpret_cast<const uint16_t*>(acc_in) + bp.nc * g.D * plane : ync,
                ACC ? static_cast<uint32_t>(g.D * plane * 2) : 0u);
  int ch_off[NCH];  // byte offset inside a plane (EW: element index), or -1 outside the plane
  int ch_lds[NCH];  // LDS element offset
  int ch_val[NCH];  // EW: elements of the chunk inside the row (1..8)
#pragma unroll
  for (int u = 0; u < NCH; ++u) {
    const int e = threadIdx.x + u * kThreads;
    ch_off[u] = -1;
    ch_lds[u] = -1;
    if (e < NCHUNK) {
      const int r = e / CPR;
      const int ch = e - r * CPR;
      const int h = th0 - P + r;
      const int w = tw0 - 8 + 8 * ch;
      ch_lds[u] = r * LC + 8 * ch;
      ch_val[u] = 0;
      if constexpr (S2 == kS2Up) {
        // Even rows only; the chunk's 8 columns hold small columns w/2 .. w/2 + 3.
        if (h >= 0 && !(h & 1) && (h >> 1) < g.Hs && w >= 0 && (w >> 1) < g.Ws)
          ch_off[u] = 2 * ((h >> 1) * g.Ws + (w >> 1));
      } else if constexpr (EW) {
        if (h >= 0 && h < g.H && w >= 0 && w < g.W) {
          ch_off[u] = h * g.W + w;
          ch_val[u] = min(8, g.W - w);
        }
      } else {
        if (h >= 0 && h < g.H && w >= 0 && w < g.W) ch_off[u] = 2 * (h * g.W + w);
      }
    }
  }
  const int nplanes = g.TD + K - 1;
  // Input plane j of this workgroup (absolute d0 - P + j); planes outside the
  // volume or past this workgroup's range read as zeros without touching memory.
  auto load_plane = [&](int j, uint4* pre, Run8* run) {
    const int di = d0 - P + j;
    if constexpr (EW && S2 == kS2Sub) {
      const bool plane_ok = j < nplanes && di >= 0 && di < g.D;
      const uint32_t pe = static_cast<uint32_t>(plane_ok ? di : 0) * static_cast<uint32_t>(plane);
#pragma unroll
      for (int u = 0; u < NCH; ++u)
        run[u] = run8_load(xr, pe + static_cast<uint32_t>(ch_off[u]), plane_ok && ch_off[u] >= 0 ? ch_val[u] : 0);
    } else if constexpr (S2 == kS2Up) {
      // Odd planes of up(small) are zero; even plane di is small plane di / 2.
      const bool plane_ok = j < nplanes && di >= 0 && !(di & 1) && (di >> 1) < g.Ds;
      const uint32_t pbase = static_cast<uint32_t>(plane_ok ? di >> 1 : 0) * static_cast<uint32_t>(splane * 2);
#pragma unroll
      for (int u = 0; u < NCH; ++u) {
        const uint32_t off = (plane_ok && ch_off[u] >= 0) ? pbase + static_cast<uint32_t>(ch_off[u]) : kOob;
        const u32x2_t v = buf_load8(xr, off);
        pre[u] = make_uint4(v[0], v[1], 0u, 0u);
      }
    } else {
      const bool plane_ok = j < nplanes && di >= 0 && di < g.D;
      const uint32_t pbase = static_cast<uint32_t>(plane_ok ? di : 0) * static_cast<uint32_t>(plane * 2);
#pragma unroll
      for (int u = 0; u < NCH; ++u) {
        const uint32_t off = (plane_ok && ch_off[u] >= 0) ? pbase + static_cast<uint32_t>(ch_off[u]) : kOob;
        pre[u] = buf_load16(xr, off);  // halo rows/planes are re-read: keep them cacheable
      }
    }
  };
  auto store_plane = [&](uint16_t* buf, const uint4* pre, const Run8* run) {
#pragma unroll
    for (int u = 0; u < NCH; ++u) {
      uint4 v;
      if constexpr (EW && S2 == kS2Sub) {
        v = run8_pack(run[u]);
      } else if constexpr (S2 == kS2Up) {
        // 4 small values -> 8 big columns, zeros at the odd ones.
        v = make_uint4(pre[u].x & 0xffffu, pre[u].x >> 16, pre[u].y & 0xffffu, pre[u].y >> 16);
      } else {
        v = pre[u];
      }
      if (ch_lds[u] >= 0) *reinterpret_cast<uint4*>(buf + ch_lds[u]) = v;
    }
  };

  f32x4_t acc[K][TPW];
#pragma unroll
  for (int s = 0; s < K; ++s)
#pragma unroll
    for (int t = 0; t < TPW; ++t) acc[s][t] = acc_init;

  constexpr bool RUNS = EW && S2 == kS2Sub;
  uint4 pre[PD][RUNS ? 1 : NCH];
  Run8 run[PD][RUNS ? NCH : 1];  // EW: the 2-byte loads of each chunk
  load_plane(0, pre[0], run[0]);
  store_plane(lds, pre[0], run[0]);
#pragma unroll
  for (int j = 1; j < PD; ++j) load_plane(j, pre[(j - 1) % PD], run[(j - 1) % PD]);
  __syncthreads();

  for (int q0 = 0; q0 < nplanes; q0 += U) {
#pragma unroll
    for (int s = 0; s < U; ++s) {
      const int i = q0 + s;
      if (i >= nplanes) break;
      load_plane(i + PD, pre[(s + PD - 1) % PD], run[(s + PD - 1) % PD]);
      const uint16_t* buf = lds + (i & 1) * LR * LC;
      const int o = i - (K - 1);  // output plane completed by this input plane
      const int cs = (s + 1) % K;
      const bool write_o = o >= 0 && o < g.TD && d0 + o < g.D && (S2 != kS2Sub || !((d0 + o) & 1));
      const uint32_t obase = S2 == kS2Sub
                                 ? static_cast<uint32_t>(write_o ? (d0 + o) >> 1 : 0) * static_cast<uint32_t>(splane * 2)
                                 : static_cast<uint32_t>(write_o ? d0 + o : 0) * static_cast<uint32_t>(plane * 2);
      // kS2Up: odd input planes are all zero; kS2Sub: odd output planes are never stored.
      const bool plane_live = S2 != kS2Up || !((d0 - P + i) & 1);
      uint16_t* const obuf = lds + 2 * LR * LC + 8 + (i & 1) * OBUF;
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int tile = wave + 4 * t;
        const int ty = tile / CT;
        const int tx = tile % CT;
        if (!plane_live) {
        } else if constexpr (BLK) {
          // Block n16 = (row n16 / 4, column n16 % 4) of the tile; lane group q
          // reads window row q (+ 4 for the second half), 8 columns from 2 to
          // the left of the block: a 4-byte aligned run.
          const uint32_t* bp0 = reinterpret_cast<const uint32_t*>(
              buf + (16 * ty + 4 * (n16 >> 2) + q) * LC + 16 * tx + 4 * (n16 & 3) + 8 - P);
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2) {
            const uint32_t* row = bp0 + h2 * 2 * LC;  // 4 rows = 4 * LC elements = 2 * LC dwords
            const uint4 raw = make_uint4(row[0], row[1], row[2], row[3]);
            const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, raw);
#pragma unroll
            for (int kd = 0; kd < K; ++kd) {
              if (S2 == kS2Sub && ((d0 + i - kd) & 1)) continue;  // odd output plane
              const int slot = ((s - kd) % K + K) % K;
              acc[slot][t] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(amat[kd][h2], bm, acc[slot][t], 0, 0, 0);
            }
          }
        } else {
          const uint16_t* bp0 = buf + (16 * ty + n16) * LC + 16 * tx + 8 * q;
#pragma unroll
          for (int kh = 0; kh < K; ++kh) {
            const bf16x8_t bm = __builtin_bit_cast(bf16x8_t, lds_read16(bp0 + kh * LC));
#pragma unroll
            for (int kd = 0; kd < K; ++kd) {
              if (S2 == kS2Sub && ((d0 + i - kd) & 1)) continue;  // odd output plane
              const int slot = ((s - kd) % K + K) % K;
              acc[slot][t] =
                  __builtin_amdgcn_mfma_f32_16x16x32_bf16(amat[kd][kh], bm, acc[slot][t], 0, 0, 0);
            }
          }
        }
        {
          const f32x4_t a = acc[cs][t];
          const bf16x4_t packed = {static_cast<__bf16>(a[0] + b0), static_cast<__bf16>(a[1] + b0),
                                   static_cast<__bf16>(a[2] + b0), static_cast<__bf16>(a[3] + b0)};
          if constexpr (STAGE) {
            *reinterpret_cast<bf16x4_t*>(obuf + (16 * ty + n16) * OC + 16 * tx + 4 * q) = packed;
          } else if constexpr (EW && S2 == kS2Up) {
            // Odd row width: the outputs inside the row, 2 bytes each.
            const int h = th0 + 16 * ty + (BLK ? 4 * (n16 >> 2) + q : n16);
            const int w = tw0 + 16 * tx + (BLK ? 4 * (n16 & 3) : 4 * q);
            const int valid = (write_o && h < g.H && w < g.W) ? min(4, g.W - w) : 0;
            const u32x2_t words = __builtin_bit_cast(u32x2_t, packed);
            const uint32_t off = obase + static_cast<uint32_t>(2 * (h * g.W + w));
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < valid) buf_store2(yr, off + 2 * e, static_cast<uint16_t>(words[e >> 1] >> (16 * (e & 1))));
          } else if constexpr (S2 == kS2Sub) {
            // Even rows keep outputs w and w + 2: small columns w / 2, w / 2 + 1.
            const int h = th0 + 16 * ty + (BLK ? 4 * (n16 >> 2) + q : n16);
            const int w = tw0 + 16 * tx + (BLK ? 4 * (n16 & 3) : 4 * q);
            const bool ok = write_o && !(h & 1) && h < g.H && w < g.W;
            const uint32_t off = ok ? obase + static_cast<uint32_t>(2 * ((h >> 1) * g.Ws + (w >> 1))) : kOob;
            const u32x2_t words = __builtin_bit_cast(u32x2_t, packed);
            buf_store4(yr, off, (words[0] & 0xffffu) | (words[1] << 16));
          } else {
            // Lane (n16, q) holds 4 consecutive outputs: 1-D, row n16 columns
            // 4 q ..; block, row 4 (n16 / 4) + q columns 4 (n16 % 4) ..
            const int h = th0 + 16 * ty + (BLK ? 4 * (n16 >> 2) + q : n16);
            const int w = tw0 + 16 * tx + (BLK ? 4 * (n16 & 3) : 4 * q);
            const bool ok = write_o && h < g.H && w < g.W;
            const uint32_t off = ok ? obase + static_cast<uint32_t>(2 * (h * g.W + w)) : kOob;
            u32x2_t words = __builtin_bit_cast(u32x2_t, packed);
            if constexpr (ACC) {
              const u32x2_t a = buf_load8(ar, off);  // zeros at the out-of-range offset
              words = u32x2_t{pack_bf16x2(bf16_lo(words[0]) + bf16_lo(a[0]), bf16_hi(words[0]) + bf16_hi(a[0])),
                              pack_bf16x2(bf16_lo(words[1]) + bf16_lo(a[1]), bf16_hi(words[1]) + bf16_hi(a[1]))};
            }
            buf_store8(yr, off, words[0], words[1]);
          }
        }
        acc[cs][t] = acc_init;
      }
      store_plane(lds + ((i + 1) & 1) * LR * LC, pre[s % PD], run[s % PD]);
      __syncthreads();
      if constexpr (STAGE) {
        // Row-contiguous store of the plane this step completed. Buffer i & 1
        // is next written at step i + 2, after the barrier that ends step i + 1.
        if (S2 == kS2Sub && write_o) {
          // Even staged rows, even columns: 8 small outputs per 16-byte store.
          constexpr int SCH = (TH / 2) * (TW / 16);
#pragma unroll
          for (int u = 0; u < (SCH + kThreads - 1) / kThreads; ++u) {
            const int e = threadIdx.x + u * kThreads;
            if (e < SCH) {
              const int r = e / (TW / 16), ch = e - r * (TW / 16);
              const int h = th0 + 2 * r, w = tw0 + 16 * ch;
              const uint16_t* src = obuf + 2 * r * OC + 16 * ch;
              const uint4 a = *reinterpret_cast<const uint4*>(src);
              const uint4 b = *reinterpret_cast<const uint4*>(src + 8);
              const uint4 v = make_uint4((a.x & 0xffffu) | (a.y << 16), (a.z & 0xffffu) | (a.w << 16),
                                         (b.x & 0xffffu) | (b.y << 16), (b.z & 0xffffu) | (b.w << 16));
              const uint32_t off =
                  (h < g.H && w < g.W) ? obase + static_cast<uint32_t>(2 * ((h >> 1) * g.Ws + (w >> 1))) : kOob;
              buf_store16(yr, off, v);
            }
          }
        } else if (EW && S2 == kS2Up && write_o) {
          // Odd row width: the staged row pieces inside the row, 2 bytes each.
#pragma unroll
          for (int u = 0; u < NOC; ++u) {
            const int e = threadIdx.x + u * kThreads;
            if (e < OCH) {
              const int r = e / (TW / 8), ch = e - r * (TW / 8);
              const int h = th0 + r, w = tw0 + 8 * ch;
              const int valid = (h < g.H && w < g.W) ? min(8, g.W - w) : 0;
              const uint16_t* src = obuf + r * OC + 8 * ch;
              const uint32_t off = obase + static_cast<uint32_t>(2 * (h * g.W + w));
#pragma unroll
              for (int el = 0; el < 8; ++el)
                if (el < valid) buf_store2(yr, off + 2 * el, src[el]);
            }
          }
        } else if (write_o) {
#pragma unroll
          for (int u = 0; u < NOC; ++u) {
            const int e = threadIdx.x + u * kThreads;
            if (e < OCH) {
              const int r = e / (TW / 8), ch = e - r * (TW / 8);
              const int h = th0 + r, w = tw0 + 8 * ch;
              const uint32_t off = (h < g.H && w < g.W) ? obase + static_cast<uint32_t>(2 * (h * g.W + w)) : kOob;
              uint4 v = *reinterpret_cast<const uint4*>(obuf + r * OC + 8 * ch);
              if constexpr (ACC) {
                const uint4 a = buf_load16(ar, off);  // zeros at the out-of-range offset
                v = make_uint4(pack_bf16x2(bf16_lo(v.x) + bf16_lo(a.x), bf16_hi(v.x) + bf16_hi(a.x)),
                               pack_bf16x2(bf16_lo(v.y) + bf16_lo(a.y), bf16_hi(v.y) + bf16_hi(a.y)),
                               pack_bf16x2(bf16_lo(v.z) + bf16_lo(a.z), bf16_hi(v.z) + bf16_hi(a.z)),
                               pack_bf16x2(bf16_lo(v.w) + bf16_lo(a.w), bf16_hi(v.w) + bf16_hi(a.w)));
              }
              buf_store16(yr, off, v);
            }
          }
        }
      }
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
// ------------------------------------------------------------- weight grad
//
// dW[kd][kh][kw] = sum_v x[d+kd-P][h+kh-P][w+kw-P] * dy[d][h][w], dB = sum_v dy.
//
// Each wave owns a block of RB = 17 - K grad_output rows and one 32-column
// unit; per x plane t its MFMA products are
//   C_{kw,kd}[i][j] += sum_{32 w} x[t][r0-P+i][w+kw-P] * dy[t-kd+P][r0+j][w]
// (i = 0..15 x rows, j < RB dy rows), so every row pair meets once and tap kh
// is the diagonal i - j = kh of C_{kw,kd}: K*K MFMAs per plane and unit, no
// tap-shifted operand copies. A workgroup (4 waves = NU units x 4/NU row
// blocks) stages each x and dy plane through LDS with row-contiguous 16-byte
// loads (double-buffered, one barrier per plane); a wave reads its x rows
// once per plane (16 bytes + the dwords either side, from which the K column
// shifts are formed in registers) and only the newly entering dy plane, the
// K most recent dy fragments rotating in registers. dB is summed from each
// dy fragment as it enters. At the end the accumulator tiles go through LDS
// and the diagonals are summed there.
template <int K, int NU>
struct WgradTile {
  static constexpr int P = K / 2;
  static constexpr int RB = 16 - 2 * P;           // grad_output rows per wave
  static constexpr int NRB = 4 / NU;               // row blocks per workgroup
  static constexpr int COLS = 32 * NU;             // columns per workgroup
  static constexpr int DROWS = RB * NRB;           // grad_output rows per workgroup
  static constexpr int XROWS = DROWS + 2 * P;      // x rows per workgroup
  static constexpr int XPITCH = COLS + 24;         // [w0-8, w0+COLS+8) + pad
  static constexpr int DPITCH = COLS + 24;
  static constexpr int XBUF = XROWS * XPITCH;      // elements
  static constexpr int DBUF = DROWS * DPITCH;
  static constexpr int XCPR = COLS / 8 + 2;        // 16-byte chunks per x row (with halo chunks)
  static constexpr int DCPR = COLS / 8;
  static constexpr int NXC = (XROWS * XCPR + kThreads - 1) / kThreads;
  static constexpr int NDC = (DROWS * DCPR + kThreads - 1) / kThreads;
  static constexpr int TILES_PER_ROUND = 3;        // accumulator tiles reduced per LDS round
  static constexpr size_t LOOP_BYTES = (2 * static_cast<size_t>(XBUF) + 2 * DBUF) * 2;  // double-buffered x and dy planes
  static constexpr size_t RED_BYTES = static_cast<size_t>(4) * TILES_PER_ROUND * 256 * 4;
  static constexpr size_t BYTES = LOOP_BYTES > RED_BYTES ? LOOP_BYTES : RED_BYTES;
};

struct WGeom {
  int C, D, H, W;
  int TD;              // grad_output planes per D-chunk
  int nDc, nRBG, nCG;  // D-chunks, row-block groups, column groups per (n, c)
  int nRB, nCU;        // row blocks (nRBG * 4 / NU) and 32-column units (nCG * NU)
  int Ds, Hs, Ws;      // UPDY: the small grad tensor dy = up(small)
};

// UPDY (the stride-2 weight gradient): dy is the small tensor read as
// up(small) on the big grid (zero at odd planes, rows and columns); the MFMAs
// of the all-zero odd dy planes are skipped.
// EW: x rows of odd width (the up block's 2s - 1 grad_output), read with
// run8_load / run8_pack.
template <int K, int NU, int PD, bool UPDY = false, bool EW = false>
__global__ __launch_bounds__(kThreads) void dw_mfma_wgrad_kernel(const bf16_t* __restrict__ x,
                                                                 const bf16_t* __restrict__ dy,
                                                                 float* __restrict__ partial,
                                                                 WGeom g, int splits) {
  using T = WgradTile<K, NU>;
  constexpr int P = T::P, RB = T::RB, K2 = K * K, K3 = K2 * K;
  extern __shared__ __align__(16) unsigned char smem_raw[];
  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem_raw);
  uint16_t* const dlds = lds + 2 * T::XBUF;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n16 = lane & 15, q = lane >> 4;
  int64_t rest = xcd_swizzle(blockIdx.x, gridDim.x);
  const int cg = static_cast<int>(rest % g.nCG);
  rest /= g.nCG;
  const int rbg = static_cast<int>(rest % g.nRBG);
  rest /= g.nRBG;
  const int dc = static_cast<int>(rest % g.nDc);
  const int64_t nc = rest / g.nDc;
  const int c = static_cast<int>(nc % g.C);
  const int64_t n = nc / g.C;
  const int r0 = rbg * T::DROWS, w0 = cg * T::COLS, d0 = dc * g.TD;
  const int dend = min(d0 + g.TD, g.D);
  const int64_t plane = static_cast<int64_t>(g.H) * g.W;
  const uint32_t plane_bytes = static_cast<uint32_t>(plane * 2);
  const __amdgpu_buffer_rsrc_t xr =
      slab_rsrc(reinterpret_cast<const uint16_t*>(x) + nc * g.D * plane, static_cast<uint32_t>(g.D) * plane_bytes);
  const int64_t splane = static_cast<int64_t>(g.Hs) * g.Ws;
  const uint32_t splane_bytes = static_cast<uint32_t>(splane * 2);
  const int64_t dslab = UPDY ? g.Ds * splane : g.D * plane;
  const __amdgpu_buffer_rsrc_t dr =
      slab_rsrc(reinterpret_cast<const uint16_t*>(dy) + nc * dslab, static_cast<uint32_t>(dslab * 2));

  // Fill chunks (same for every plane): x rows r0-P .. r0+DROWS+P-1, columns
  // [w0-8, w0+COLS+8) in 8-element chunks; dy rows r0 .. r0+DROWS-1, columns
  // [w0, w0+COLS). Byte offsets inside a plane, -1 outside it.
  int xg[T::NXC], xl[T::NXC], dg[T::NDC], dl[T::NDC];
  int xv[EW ? T::NXC : 1];  // EW: elements of the chunk inside the row
#pragma unroll
  for (int u = 0; u < T::NXC; ++u) {
    const int e = threadIdx.x + u * kThreads;
    xg[u] = -1;
    xl[u] = -1;
    if constexpr (EW) xv[u] = 0;
    if (e < T::XROWS * T::XCPR) {
      const int r = e / T::XCPR, ch = e - r * T::XCPR;
      const int h = r0 - P + r, w = w0 - 8 + 8 * ch;
      xl[u] = r * T::XPITCH + 8 * ch;
      if (h >= 0 && h < g.H && w >= 0 && w < g.W) {
        if constexpr (EW) {
          xg[u] = h * g.W + w;  // element index
          xv[u] = min(8, g.W - w);
        } else {
          xg[u] = 2 * (h * g.W + w);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < T::NDC; ++u) {
    const int e = threadIdx.x + u * kThreads;
    dg[u] = -1;
    dl[u] = -1;
    if (e < T::DROWS * T::DCPR) {
      const int r = e / T::DCPR, ch = e - r * T::DCPR;
      const int h = r0 + r, w = w0 + 8 * ch;
      dl[u] = r * T::DPITCH + 8 * ch;
      if constexpr (UPDY) {
        // Even rows only; the chunk's 8 columns hold small columns w/2 .. w/2 + 3.
        if (!(h & 1) && (h >> 1) < g.Hs && (w >> 1) < g.Ws) dg[u] = 2 * ((h >> 1) * g.Ws + (w >> 1));
      } else {
        if (h < g.H && w < g.W) dg[u] = 2 * (h * g.W + w);
      }
    }
  }

  // Step s: x plane t = d0 - P + s, and grad_output plane t + P (which enters
  // the ring); each is zero outside its valid range.
  const int nsteps = (dend - d0) + 2 * P;
  struct Pre {
    uint4 xv[EW ? 1 : T::NXC];
    uint4 dv[T::NDC];
    Run8 xr8[EW ? T::NXC : 1];  // EW: the 2-byte loads of each x chunk
  };
  auto load = [&](int s, Pre& p) {
    const int t = d0 - P + s;
    const bool xok = s < nsteps && t >= 0 && t < g.D;
    const uint32_t xb = static_cast<uint32_t>(xok ? t : 0) * plane_bytes;
    const int td = t + P;
    const bool dok = s < nsteps && td >= d0 && td < dend && (!UPDY || (!(td & 1) && (td >> 1) < g.Ds));
    const uint32_t dbo = UPDY ? static_cast<uint32_t>(dok ? td >> 1 : 0) * splane_bytes
                              : static_cast<uint32_t>(dok ? td : 0) * plane_bytes;
#pragma unroll
    for (int u = 0; u < T::NXC; ++u) {
      if constexpr (EW) {
        const uint32_t pe = static_cast<uint32_t>(xok ? t : 0) * static_cast<uint32_t>(plane);
        p.xr8[u] = run8_load(xr, pe + static_cast<uint32_t>(xg[u]), xok && xg[u] >= 0 ? xv[u] : 0);
      } else {
        p.xv[u] = buf_load16(xr, xok && xg[u] >= 0 ? xb + xg[u] : kOob);
      }
    }
#pragma unroll
    for (int u = 0; u < T::NDC; ++u) {
      const uint32_t off = dok && dg[u] >= 0 ? dbo + dg[u] : kOob;
      if constexpr (UPDY) {
        const u32x2_t v = buf_load8(dr, off);
        p.dv[u] = make_uint4(v[0], v[1], 0u, 0u);
      } else {
        p.dv[u] = buf_load16_nt(dr, off);
      }
    }
  };
  auto store = [&](int s, const Pre& p) {
    uint16_t* const xb = lds + (s & 1) * T::XBUF;
    uint16_t* const db = dlds + (s & 1) * T::DBUF;
#pragma unroll
    for (int u = 0; u < T::NXC; ++u) {
      uint4 v;
      if constexpr (EW) {
        v = run8_pack(p.xr8[u]);
      } else {
        v = p.xv[u];
      }
      if (xl[u] >= 0) *reinterpret_cast<uint4*>(xb + xl[u]) = v;  // masked off without a chunk
    }
#pragma unroll
    for (int u = 0; u < T::NDC; ++u) {
      uint4 v = p.dv[u];
      // UPDY: 4 small values -> 8 big columns, zeros at the odd ones.
      if constexpr (UPDY) v = make_uint4(v.x & 0xffffu, v.x >> 16, v.y & 0xffffu, v.y >> 16);
      if (dl[u] >= 0) *reinterpret_cast<uint4*>(db + dl[u]) = v;
    }
  };

  // This wave: unit u0 (32 columns), row block j0 of the workgroup.
  const int u0 = wave % NU, j0 = wave / NU;
  const int a_row = (j0 * RB + n16) * T::XPITCH + 8 + 32 * u0 + 8 * q;  // x row j0*RB + n16 (tile row = x row - r0 + P)
  const bool b_ok = n16 < RB;
  const int b_row = (j0 * RB + (b_ok ? n16 : 0)) * T::DPITCH + 32 * u0 + 8 * q;

  f32x4_t acc[K][K];
#pragma unroll
  for (int a = 0; a < K; ++a)
#pragma unroll
    for (int b = 0; b < K; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4 ring[K];  // ring[kd] = dy fragment of plane t - kd + P
#pragma unroll
  for (int kd = 0; kd < K; ++kd) ring[kd] = make_uint4(0u, 0u, 0u, 0u);
  float dbias = 0.f;

  Pre pre[PD];
  {
    Pre first;
    load(0, first);
    store(0, first);
  }
#pragma unroll
  for (int j = 1; j < PD; ++j) load(j, pre[(j - 1) % PD]);
  __syncthreads();

  for (int s0 = 0; s0 < nsteps; s0 += PD) {
#pragma unroll
    for (int jj = 0; jj < PD; ++jj) {
      const int st = s0 + jj;
      if (st >= nsteps) break;
      load(st + PD, pre[(jj + PD - 1) % PD]);
      const uint16_t* const xb = lds + (st & 1) * T::XBUF;
      const uint16_t* const db = dlds + (st & 1) * T::DBUF;
      uint4 bnew = make_uint4(0u, 0u, 0u, 0u);
      if (b_ok) bnew = lds_read16(db + b_row);
      const uint4 xm = lds_read16(xb + a_row);
      const uint32_t xp = *reinterpret_cast<const uint32_t*>(xb + a_row - 2);
      const uint32_t xn = *reinterpret_cast<const uint32_t*>(xb + a_row + 8);
#pragma unroll
      for (int kd = K - 1; kd > 0; --kd) ring[kd] = ring[kd - 1];
      ring[0] = bnew;
      dbias += (bf16_lo(bnew.x) + bf16_hi(bnew.x)) + (bf16_lo(bnew.y) + bf16_hi(bnew.y)) +
               (bf16_lo(bnew.z) + bf16_hi(bnew.z)) + (bf16_lo(bnew.w) + bf16_hi(bnew.w));
      // Words of x[col-2 .. col+9]; shift sh = kw - P selects x[col+sh .. col+sh+7].
      const uint32_t e[6] = {xp, xm.x, xm.y, xm.z, xm.w, xn};
#pragma unroll
      for (int kw = 0; kw < K; ++kw) {
        const int sh = kw - P;
        uint4 av;
        if (sh % 2 == 0) {
          const int b = 1 + sh / 2;
          av = make_uint4(e[b], e[b + 1], e[b + 2], e[b + 3]);
        } else {
          const int b = sh < 0 ? 0 : 1;  // |sh| == 1
          av = make_uint4(__builtin_amdgcn_alignbit(e[b + 1], e[b], 16),
                          __builtin_amdgcn_alignbit(e[b + 2], e[b + 1], 16),
                          __builtin_amdgcn_alignbit(e[b + 3], e[b + 2], 16),
                          __builtin_amdgcn_alignbit(e[b + 4], e[b + 3], 16));
        }
#pragma unroll
        for (int kd = 0; kd < K; ++kd) {
          if (UPDY && ((d0 + st - kd) & 1)) continue;  // ring[kd] holds dy plane d0 + st - kd: odd = zero
          acc[kw][kd] = mfma16x16x32(av, ring[kd], acc[kw][kd]);
        }
      }
      store(st + 1, pre[jj % PD]);
      __syncthreads();
    }
  }

  // Diagonal sums through LDS, TILES_PER_ROUND accumulator tiles per round.
  // Tile (kw, kd) of wave w: red[(w * TILES + tile) * 256 + i * 16 + j] = C[i][j];
  // tap (kd, kh, kw) = sum_{j < RB} C[j + kh][j].
  const int64_t rb = static_cast<int64_t>(rbg) * T::NRB + j0;
  const int64_t cu = static_cast<int64_t>(cg) * NU + u0;
  const int64_t split = ((n * g.nDc + dc) * g.nRB + rb) * g.nCU + cu;
  float* const out = partial + static_cast<int64_t>(c) * (K3 + 1) * splits;
  float* const red = reinterpret_cast<float*>(smem_raw);
  constexpr int TPR = T::TILES_PER_ROUND;
  const float dbt = wave_sum(dbias);
  if (lane == 0) out[static_cast<int64_t>(K3) * splits + split] = dbt;
#pragma unroll
  for (int base = 0; base < K2; base += TPR) {
#pragma unroll
    for (int tt = 0; tt < TPR; ++tt) {
      const int tile = base + tt;
      if (tile < K2) {
        const int kw = tile / K, kd = tile % K;
#pragma unroll
        for (int r = 0; r < 4; ++r) red[(wave * TPR + tt) * 256 + (4 * q + r) * 16 + n16] = acc[kw][kd][r];
      }
    }
    __syncthreads();
    // One thread per (wave, tile, kh) sums RB diagonal entries in order.
    for (int e = threadIdx.x; e < 4 * TPR * K; e += kThreads) {
      const int w = e / (TPR * K), rem = e % (TPR * K), tt = rem / K, kh = rem % K;
      const int tile = base + tt;
      if (tile < K2) {
        const int kw = tile / K, kd = tile % K;
        const float* tp = red + (w * TPR + tt) * 256;
        float v = 0.f;
        for (int j = 0; j < RB; ++j) v += tp[(j + kh) * 16 + j];
        const int64_t wrb = static_cast<int64_t>(rbg) * T::NRB + w / NU;
        const int64_t wcu = static_cast<int64_t>(cg) * NU + w % NU;
        const int64_t wsplit = ((n * g.nDc + dc) * g.nRB + wrb) * g.nCU + wcu;
        out[static_cast<int64_t>(kd * K2 + kh * K + kw) * splits + wsplit] = v;
      }
    }
    __syncthreads();
  }
}

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
                   int64_t blocks, hipStream_t st, const void* acc = nullptr) {
  constexpr int P = K / 2;
  // two plane buffers, 8 spare elements, then (k = 3) the output staging tile
  constexpr size_t stage = stencil_stages_output(K) ? static_cast<size_t>(2) * (16 * kRT) * (16 * CT + 8) : 0;
  constexpr size_t lds = (static_cast<size_t>(2) * (16 * kRT + 2 * P) * stencil_pitch(K, CT) + 8 + stage) * 2;
  auto px = static_cast<const bf16_t*>(x);
  auto pw = static_cast<const bf16_t*>(wt);
  auto pb = static_cast<const bf16_t*>(bias);
  auto py = static_cast<bf16_t*>(y);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
  if constexpr (FLIP) {
    if (acc != nullptr) {
      hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, false, CT, PD, true>), grid, block, lds, st, px, pw,
                         pb, py, g, static_cast<const bf16_t*>(acc));
      MEDNEXT_CHECK_LAUNCH();
      return MEDNEXT_STATUS_OK;
    }
  }
  if (bias)
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, true, CT, PD>), grid, block, lds, st, px,
                       pw, pb, py, g);
  else
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, false, CT, PD>), grid, block, lds, st, px,
                       pw, pb, py, g);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

// Stride-2 maps on the stencil: kS2Sub (gather: forward taps over big, small
// output) or kS2Up (scatter: flipped taps over up(small), big output).
template <int K, int S2, int CT, bool EW>
int launch_stencil_s2(const void* x, const void* wt, const void* bias, void* y, const MGeom& g, int64_t blocks,
                      hipStream_t st) {
  constexpr int P = K / 2;
  constexpr int PD = K == 3 && !(EW && S2 == kS2Sub) ? 4 : 2;  // 2-byte runs hold 8 registers per chunk
  constexpr bool FLIP = S2 == kS2Up;
  constexpr size_t stage = stencil_stages_output(K) ? static_cast<size_t>(2) * (16 * kRT) * (16 * CT + 8) : 0;
  constexpr size_t lds = (static_cast<size_t>(2) * (16 * kRT + 2 * P) * stencil_pitch(K, CT) + 8 + stage) * 2;
  auto px = static_cast<const bf16_t*>(x);
  auto pw = static_cast<const bf16_t*>(wt);
  auto pb = static_cast<const bf16_t*>(bias);
  auto py = static_cast<bf16_t*>(y);
  const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
  if (bias)
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, true, CT, PD, false, S2, EW>), grid, block, lds, st, px, pw,
                       pb, py, g, nullptr);
  else
    hipLaunchKernelGGL((dw_mfma_stencil_kernel<K, FLIP, false, CT, PD, false, S2, EW>), grid, block, lds, st, px, pw,
                       pb, py, g, nullptr);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <int K, int S2, bool EW>
int launch_stencil_s2_ct(const void* x, const void* wt, const void* bias, void* y, const MGeom& g, int tile_cols,
                         int64_t blocks, hipStream_t st) {
  switch (tile_cols) {
    case 32: return launch_stencil_s2<K, S2, 2, EW>(x, wt, bias, y, g, blocks, st);
    case 64: return launch_stencil_s2<K, S2, 4, EW>(x, wt, bias, y, g, blocks, st);
    default: return launch_stencil_s2<K, S2, 8, EW>(x, wt, bias, y, g, blocks, st);
  }
}

template <int S2>
int launch_stencil_s2_k(const void* x, const void* wt, const void* bias, void* y, const MGeom& g, int k, bool ew,
                        int tile_cols, int64_t blocks, hipStream_t st) {
  if (k == 3)
    return ew ? launch_stencil_s2_ct<3, S2, true>(x, wt, bias, y, g, tile_cols, blocks, st)
              : launch_stencil_s2_ct<3, S2, false>(x, wt, bias, y, g, tile_cols, blocks, st);
  return ew ? launch_stencil_s2_ct<5, S2, true>(x, wt, bias, y, g, tile_cols, blocks, st)
            : launch_stencil_s2_ct<5, S2, false>(x, wt, bias, y, g, tile_cols, blocks, st);
}

template <int K, bool FLIP>
int launch_stencil_ct(const void* x, const void* wt, const void* bias, void* y, const MGeom& g,
                      int tile_cols, int64_t blocks, hipStream_t st, const void* acc) {
  constexpr int PD = K == 3 ? 4 : 2;
  switch (tile_cols) {
    case 32: return launch_stencil<K, FLIP, 2, PD>(x, wt, bias, y, g, blocks, st, acc);
    case 64: return launch_stencil<K, FLIP, 4, PD>(x, wt, bias, y, g, blocks, st, acc);
    default: return launch_stencil<K, FLIP, 8, PD>(x, wt, bias, y, g, blocks, st, acc);
  }
}


template <int K, int NU, bool UPDY = false, bool EW = false>
int launch_wgrad(const void* x, const void* dy, float* partial, const WGeom& g, int64_t blocks, int splits,
                 hipStream_t st) {
  constexpr int PD = 2;
  const size_t lds = WgradTile<K, NU>::BYTES;
  hipLaunchKernelGGL((dw_mfma_wgrad_kernel<K, NU, PD, UPDY, EW>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kThreads), lds, st, static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(dy), partial,
                     g, splits);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <bool UPDY, bool EW = false>
int launch_wgrad_k(const void* x, const void* dy, float* partial, const WGeom& g, int k, int tile_cols,
                   int64_t blocks, int splits, hipStream_t st) {
  if (k == 3) {
    switch (tile_cols) {
      case 32: return launch_wgrad<3, 1, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
      case 64: return launch_wgrad<3, 2, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
      default: return launch_wgrad<3, 4, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
    }
  }
  switch (tile_cols) {
    case 32: return launch_wgrad<5, 1, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
    case 64: return launch_wgrad<5, 2, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
    default: return launch_wgrad<5, 4, UPDY, EW>(x, dy, partial, g, blocks, splits, st);
  }
}

// any_width: the caller has checked the shape (the stride-2 form, whose big
// rows may have odd width).
int plan_wgrad(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int tile_cols,
               int depth_chunk, WGeom* g, int64_t* blocks, int* splits, bool any_width = false) {
  MEDNEXT_CHECK_ARG(any_width || (dw_mfma_supported(d, h, w, k) && w % 32 == 0),
                    "MFMA wgrad needs k in {3,5}, W % 32 == 0, H >= 32 and a slab < 2 GiB");
  MEDNEXT_CHECK_ARG(tile_cols == 32 || tile_cols == 64 || tile_cols == 128,
                    "MFMA wgrad tile_w (columns per workgroup) must be 32, 64 or 128");
  MEDNEXT_CHECK_ARG(depth_chunk >= 1, "depth_chunk must be >= 1");
  const int nu = tile_cols / 32;
  const int rb = 16 - 2 * (k / 2);
  g->C = static_cast<int>(c);
  g->D = static_cast<int>(d);
  g->H = static_cast<int>(h);
  g->W = static_cast<int>(w);
  g->TD = static_cast<int>(depth_chunk < d ? depth_chunk : d);
  g->nDc = static_cast<int>(cdiv(d, g->TD));
  g->nRBG = static_cast<int>(cdiv(h, static_cast<int64_t>(rb) * (4 / nu)));
  g->nCG = static_cast<int>(cdiv(w, tile_cols));
  g->nRB = g->nRBG * (4 / nu);
  g->nCU = g->nCG * nu;
  const int64_t per_channel = static_cast<int64_t>(g->nDc) * g->nRBG * g->nCG;
  *blocks = n * c * per_channel;
  const int64_t sp = n * static_cast<int64_t>(g->nDc) * g->nRB * g->nCU;
  MEDNEXT_CHECK_ARG(*blocks < (int64_t(1) << 31) && sp < (int64_t(1) << 31), "grid too large");
  *splits = static_cast<int>(sp);
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
                    int depth_chunk, hipStream_t st, const void* acc) {
  MEDNEXT_CHECK_ARG(acc == nullptr || flip, "accumulation is for the input gradient");
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
    return flip ? launch_stencil_ct<3, true>(x, weight, bias, y, g, tile_cols, blocks, st, acc)
                : launch_stencil_ct<3, false>(x, weight, bias, y, g, tile_cols, blocks, st, nullptr);
  }
  return flip ? launch_stencil_ct<5, true>(x, weight, bias, y, g, tile_cols, blocks, st, acc)
              : launch_stencil_ct<5, false>(x, weight, bias, y, g, tile_cols, blocks, st, nullptr);
}


int dw_mfma_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k,
                         int tile_cols, int depth_chunk) {
  WGeom g{};
  int64_t blocks = 0;
  int splits = 0;
  if (plan_wgrad(n, c, d, h, w, k, tile_cols, depth_chunk, &g, &blocks, &splits) != MEDNEXT_STATUS_OK) return 0;
  return splits;
}

int dw_mfma_wgrad(const void* x, const void* dy, float* partial, int64_t n, int64_t c, int64_t d,
                  int64_t h, int64_t w, int k, int tile_cols, int depth_chunk, hipStream_t st) {
  WGeom g{};
  int64_t blocks = 0;
  int splits = 0;
  const int status = plan_wgrad(n, c, d, h, w, k, tile_cols, depth_chunk, &g, &blocks, &splits);
  if (status != MEDNEXT_STATUS_OK) return status;
  return launch_wgrad_k<false>(x, dy, partial, g, k, tile_cols, blocks, splits, st);
}

// ------------------------------------------------------------------ stride 2

namespace {

// Launch shapes of the stride-2 maps (no recipe argument: the entry points
// keep the reference's signature). Stencil: the widest tile the row allows and
// D-runs for ~2 workgroups per CU, as for the stride-1 stencil. Weight
// gradient: the stride-1 weight gradient's targets (2.5 workgroups per CU for
// k = 3; for k = 5 at most 2).
constexpr int64_t kS2StencilTarget = 2 * 256;

int s2_tile_cols(int64_t wb) { return wb >= 128 ? 128 : wb >= 64 ? 64 : 32; }

// within: at most `target` workgroups (the k = 5 weight gradient, two resident
// per CU, whose partial second round costs about as much as a full one)
// instead of at least.
int s2_depth_chunk(int64_t db, int64_t slabs, int64_t target, bool within = false) {
  const int64_t sl = std::max<int64_t>(1, slabs);
  const int64_t chunks = std::max<int64_t>(1, within ? target / sl : cdiv(target, sl));
  return static_cast<int>(std::max<int64_t>(2, cdiv(db, chunks)));
}

int s2_stencil_geom(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                    MGeom* g, int* tile_cols, int64_t* blocks) {
  *tile_cols = s2_tile_cols(wb);
  const int64_t slabs = n * c * cdiv(hb, int64_t(16 * kRT)) * cdiv(wb, int64_t(*tile_cols));
  if (int st = make_geom(c, db, hb, wb, *tile_cols, s2_depth_chunk(db, slabs, kS2StencilTarget), g)) return st;
  g->Ds = static_cast<int>(ds);
  g->Hs = static_cast<int>(hs);
  g->Ws = static_cast<int>(ws);
  *blocks = n * c * g->nDc * g->nHt * g->nWt;
  MEDNEXT_CHECK_ARG(*blocks < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

int s2_wgrad_geom(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                  int k, WGeom* g, int* tile_cols, int64_t* blocks, int* splits) {
  *tile_cols = s2_tile_cols(wb);
  const int64_t rows = int64_t(16 - (k - 1)) * (4 / (*tile_cols / 32));
  const int64_t slabs = n * c * cdiv(hb, rows) * cdiv(wb, int64_t(*tile_cols));
  const int64_t target = k == 3 ? 5 * 256 / 2 : 2 * 256;
  const int dc = s2_depth_chunk(db, slabs, target, k == 5);
  if (int st = plan_wgrad(n, c, db, hb, wb, k, *tile_cols, dc, g, blocks, splits, true)) return st;
  g->Ds = static_cast<int>(ds);
  g->Hs = static_cast<int>(hs);
  g->Ws = static_cast<int>(ws);
  return MEDNEXT_STATUS_OK;
}

}  // namespace

bool dw_mfma_s2_supported(int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k) {
  // Big = 2 * small (the down block) or 2 * small - 1 (the up block's output)
  // per dimension. Even big rows: W % 32 == 0 (whole weight-gradient units,
  // aligned 16-byte row pieces); odd big rows (element-exact access): small
  // rows of whole 8-column pieces. Both: H, W >= 32 and a slab < 2 GiB.
  auto pair = [](int64_t b, int64_t s) { return b == 2 * s || b == 2 * s - 1; };
  const bool width = wb % 2 == 0 ? wb % 32 == 0 : ws % 8 == 0;
  return (k == 3 || k == 5) && pair(db, ds) && pair(hb, hs) && pair(wb, ws) && width && hb >= 32 && wb >= 32 &&
         db * hb * wb * 2 < (int64_t(1) << 31) && ds * hs * ws * 2 < (int64_t(1) << 31);
}

int dw_mfma_s2_gather(const void* big, const void* weight, const void* bias, void* small, int64_t n, int64_t c,
                      int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st) {
  MEDNEXT_CHECK_ARG(dw_mfma_s2_supported(db, hb, wb, ds, hs, ws, k), "shape not supported by the MFMA stride-2 maps");
  MGeom g{};
  int tile_cols = 0;
  int64_t blocks = 0;
  if (int s = s2_stencil_geom(n, c, db, hb, wb, ds, hs, ws, &g, &tile_cols, &blocks)) return s;
  return launch_stencil_s2_k<kS2Sub>(big, weight, bias, small, g, k, wb % 2 != 0, tile_cols, blocks, st);
}

int dw_mfma_s2_scatter(const void* small, const void* weight, const void* bias, void* big, int64_t n, int64_t c,
                       int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st) {
  MEDNEXT_CHECK_ARG(dw_mfma_s2_supported(db, hb, wb, ds, hs, ws, k), "shape not supported by the MFMA stride-2 maps");
  MGeom g{};
  int tile_cols = 0;
  int64_t blocks = 0;
  if (int s = s2_stencil_geom(n, c, db, hb, wb, ds, hs, ws, &g, &tile_cols, &blocks)) return s;
  return launch_stencil_s2_k<kS2Up>(small, weight, bias, big, g, k, wb % 2 != 0, tile_cols, blocks, st);
}

int dw_mfma_s2_wgrad_splits(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                            int64_t ws, int k) {
  if (!dw_mfma_s2_supported(db, hb, wb, ds, hs, ws, k)) return 0;
  WGeom g{};
  int tile_cols = 0, splits = 0;
  int64_t blocks = 0;
  if (s2_wgrad_geom(n, c, db, hb, wb, ds, hs, ws, k, &g, &tile_cols, &blocks, &splits) != MEDNEXT_STATUS_OK) return 0;
  return splits;
}

int dw_mfma_s2_wgrad(const void* big, const void* small, float* partial, int64_t n, int64_t c, int64_t db, int64_t hb,
                     int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st) {
  MEDNEXT_CHECK_ARG(dw_mfma_s2_supported(db, hb, wb, ds, hs, ws, k), "shape not supported by the MFMA stride-2 maps");
  WGeom g{};
  int tile_cols = 0, splits = 0;
  int64_t blocks = 0;
  if (int s = s2_wgrad_geom(n, c, db, hb, wb, ds, hs, ws, k, &g, &tile_cols, &blocks, &splits)) return s;
  return wb % 2 != 0 ? launch_wgrad_k<true, true>(big, small, partial, g, k, tile_cols, blocks, splits, st)
                     : launch_wgrad_k<true, false>(big, small, partial, g, k, tile_cols, blocks, splits, st);
}

}  // namespace mednext
