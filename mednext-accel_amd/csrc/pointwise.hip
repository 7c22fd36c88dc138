// bf16 1x1x1 (pointwise) convolutions on CDNA4 matrix cores, with the MedNeXt
// block's elementwise work fused into the GEMMs.
//
// A 1x1x1 conv of an NCDHW tensor is, per sample, Y[M][V] = W[M][K] . X[K][V]
// (+ b[M]) with V = D*H*W voxels contiguous in memory and the K (= input
// channel) rows V elements apart.
//
// Forward / input-gradient (pw_fwd_kernel). v_mfma_f32_16x16x32_bf16 wants, per
// lane, 8 consecutive K values of one output column. Instead of transposing X
// through LDS, a wave maps MFMA output column n of its j-th MFMA (j = 0..7) to
// voxel v0 + 8n + j: lane (q = l/16, n = l%16) then needs X[k0+8q+i][v0+8n+j]
// for i, j in 0..7, which is exactly the 8x8 block it gets from eight 16-byte
// loads (one per channel row k0+8q+i, voxels v0+8n .. v0+8n+7). An in-register
// 8x8 transpose (32 v_perm_b32) forms the eight B operands; no LDS traffic and
// every global load is 16 bytes. The accumulators come out as
// C[4q+r][n] of MFMA j = Y[m][v0+8n+j]: for each row a lane holds 8 consecutive
// voxels, so the epilogue stores 16 bytes per row as well. The weight block
// (64 output rows x K) sits in LDS in A-fragment order, transposed on load for
// the input gradient (A = W^T).
// Fused epilogues: + bias; + bias then GELU; + bias + residual; x GELU'(h)
// (input gradient of project followed by the GELU backward). Fused prologue:
// GELU on the loaded X (the project GEMM reads the expand pre-activation h and
// recomputes GELU(h) instead of storing it).
//
// Weight gradient (pw_wgrad_kernel). dW[M][K] = sum_v dY[M][v] . X[K][v] reduces
// over the contiguous V axis, so both operands load naturally (A = 8
// consecutive voxels of a dY row, B = 8 consecutive voxels of an X row).
// dB[m] = sum_v dY[m][v] is accumulated from the same A fragments on the VALU.
// Each workgroup writes a deterministic fp32 partial of its V range; a finish
// kernel sums the partials in a fixed order in fp64.
//
// GELU is the exact (erf) form. erf uses Abramowitz & Stegun, Handbook of
// Mathematical Functions, eq. 7.1.26 (|error| <= 1.5e-7), far below the bf16
// rounding the results get.
#include <algorithm>

#include "cdna4.h"
#include "common.h"

namespace mednext {
namespace {

constexpr int kPwThreads = 256;  // 4 waves
constexpr int kPwMT = 4;         // 16-row m-tiles per workgroup -> 64 output rows
constexpr int kPwRows = 16 * kPwMT;
constexpr int kChunk = 128;      // voxels per wave step (16 columns x 8 MFMAs)
constexpr int kMaxK = 512;       // LDS weight block: 64 x K bf16 <= 64 KiB

struct PwGeom {
  int K, M;          // GEMM reduction and output rows
  uint32_t V;        // voxels per sample
  int chunks;        // ceil(V / kChunk)
  int wt;            // 1: weight stored [K][M] (A = W^T), 0: [M][K]
};

__device__ inline float erf_as(float x) {
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(0.3275911f, ax, 1.0f));
  float p = fmaf(1.061405429f, t, -1.453152027f);
  p = fmaf(p, t, 1.421413741f);
  p = fmaf(p, t, -0.284496736f);
  p = fmaf(p, t, 0.254829592f);
  p *= t;
  const float r = 1.0f - p * __expf(-ax * ax);
  return copysignf(r, x);
}

__device__ inline float gelu_f(float h) { return 0.5f * h * (1.0f + erf_as(h * 0.7071067811865476f)); }

// d/dh of h * Phi(h) = Phi(h) + h * phi(h).
__device__ inline float gelu_grad_f(float h) {
  const float cdf = 0.5f * (1.0f + erf_as(h * 0.7071067811865476f));
  return fmaf(h * 0.3989422804014327f, __expf(-0.5f * h * h), cdf);
}

__device__ inline uint32_t gelu_word(uint32_t w) {
  return pack_bf16x2(gelu_f(bf16_lo(w)), gelu_f(bf16_hi(w)));
}
__device__ inline uint4 gelu_vec(uint4 v) {
  return make_uint4(gelu_word(v.x), gelu_word(v.y), gelu_word(v.z), gelu_word(v.w));
}

__device__ inline uint32_t word(const uint4& v, int d) {
  return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
}

// raw[i] = 8 voxels (j) of channel row i; returns bv[j] = 8 channels (i) of voxel j.
__device__ inline void transpose8x8(const uint4 (&raw)[8], uint4 (&bv)[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {  // voxel pair (2d, 2d+1)
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // channel pair (2p, 2p+1)
      const uint32_t a = word(raw[2 * p], d), b = word(raw[2 * p + 1], d);
      lo[p] = __builtin_amdgcn_perm(b, a, 0x05040100u);  // (a.lo, b.lo): voxel 2d
      hi[p] = __builtin_amdgcn_perm(b, a, 0x07060302u);  // (a.hi, b.hi): voxel 2d+1
    }
    bv[2 * d] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    bv[2 * d + 1] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  }
}

// Weight block [m0, m0 + 64) x [0, K) into LDS in A-fragment order: fragment
// (ks, mt) is 64 lanes x 16 bytes at ((ks * kPwMT + mt) * 64 + lane) * 16.
__device__ void load_weight_block(const bf16_t* __restrict__ w, uint16_t* lds, const PwGeom& g, int m0) {
  const int tid = threadIdx.x;
  if (!g.wt) {
    const int per_row = g.K / 8;
    for (int p = tid; p < kPwRows * per_row; p += kPwThreads) {
      const int r = p / per_row, k8 = (p % per_row) * 8;
      const int m = m0 + r;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m < g.M) v = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(m) * g.K + k8);
      const int ks = k8 / 32, q = (k8 % 32) / 8, mt = r / 16, c = r % 16;
      *reinterpret_cast<uint4*>(lds + (((ks * kPwMT + mt) * 64) + q * 16 + c) * 8) = v;
    }
  } else {  // w is [K][M]: A[m][k] = w[k][m]
    for (int p = tid; p < g.K * (kPwRows / 8); p += kPwThreads) {
      const int k = p / (kPwRows / 8), mg = (p % (kPwRows / 8)) * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + mg < g.M) v = *reinterpret_cast<const uint4*>(w + static_cast<int64_t>(k) * g.M + m0 + mg);
      const int ks = k / 32, q = (k % 32) / 8, i = k % 8;
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int r = mg + jj, mt = r / 16, c = r % 16;
        const uint32_t wd = word(v, jj / 2);
        lds[(((ks * kPwMT + mt) * 64) + q * 16 + c) * 8 + i] = static_cast<uint16_t>((jj & 1) ? (wd >> 16) : wd);
      }
    }
  }
}

template <int PRO, int EPI>
__global__ __launch_bounds__(kPwThreads) void pw_fwd_kernel(const bf16_t* __restrict__ x,
                                                            const bf16_t* __restrict__ w,
                                                            const bf16_t* __restrict__ bias,
                                                            const bf16_t* __restrict__ aux,
                                                            bf16_t* __restrict__ y, PwGeom g) {
  extern __shared__ __align__(16) uint16_t pw_lds[];
  const int m0 = blockIdx.y * kPwRows;
  load_weight_block(w, pw_lds, g, m0);
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_col = lane & 15, q = lane >> 4;
  const int64_t n = blockIdx.z;
  const uint32_t V = g.V;
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(y + n * g.M * static_cast<int64_t>(V), g.M * V * 2u);
  const bf16_t* auxn = aux != nullptr ? aux + n * g.M * static_cast<int64_t>(V) : nullptr;
  const __amdgpu_buffer_rsrc_t ar = slab_rsrc(auxn != nullptr ? auxn : y, auxn != nullptr ? g.M * V * 2u : 0u);
  const int ksteps = g.K / 32;
  const int mtiles = min(kPwMT, (g.M - m0) / 16);
  const uint4* frag = reinterpret_cast<const uint4*>(pw_lds) + lane;

  for (int chunk = blockIdx.x * 4 + wave; chunk < g.chunks; chunk += gridDim.x * 4) {
    const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
    const bool vok = vl < V;
    f32x4_t acc[kPwMT][8];
#pragma unroll
    for (int mt = 0; mt < kPwMT; ++mt)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    uint4 raw[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) raw[i] = buf_load16(xr, vok ? ((8u * q + i) * V + vl) * 2u : kOob);
    for (int ks = 0; ks < ksteps; ++ks) {
      uint4 cur[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) cur[i] = raw[i];
      if (ks + 1 < ksteps) {  // prefetch the next 32 channels
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const uint32_t row = 32u * (ks + 1) + 8u * q + i;
          raw[i] = buf_load16(xr, vok ? (row * V + vl) * 2u : kOob);
        }
      }
      if (PRO == MEDNEXT_PW_PROLOGUE_GELU) {
#pragma unroll
        for (int i = 0; i < 8; ++i) cur[i] = gelu_vec(cur[i]);
      }
      uint4 bv[8];
      transpose8x8(cur, bv);
#pragma unroll
      for (int mt = 0; mt < kPwMT; ++mt) {
        if (mt < mtiles) {
          const uint4 a = frag[(ks * kPwMT + mt) * 64];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[mt][j] = mfma16x16x32(a, bv[j], acc[mt][j]);
        }
      }
    }

    // Epilogue: row m = m0 + 16 mt + 4 q + r, voxels vl .. vl + 7.
#pragma unroll
    for (int mt = 0; mt < kPwMT; ++mt) {
      if (mt >= mtiles) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * mt + 4 * q + r;
        const uint32_t off = vok ? (static_cast<uint32_t>(m) * V + vl) * 2u : kOob;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = acc[mt][j][r];
        if (EPI != MEDNEXT_PW_EPILOGUE_GELU_GRAD && bias != nullptr) {
          const float b = bf16_to_f32(bias[m].bits);
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] += b;
        }
        if (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = gelu_f(v[j]);
        } else if (EPI == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL || EPI == MEDNEXT_PW_EPILOGUE_GELU_GRAD) {
          const uint4 a = buf_load16(ar, off);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint32_t wd = word(a, j / 2);
            const float e = (j & 1) ? bf16_hi(wd) : bf16_lo(wd);
            v[j] = EPI == MEDNEXT_PW_EPILOGUE_GELU_GRAD ? v[j] * gelu_grad_f(e) : v[j] + e;
          }
        }
        buf_store16(yr, off,
                    make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                               pack_bf16x2(v[6], v[7])));
      }
    }
  }
}

// ---------------------------------------------------------------- weight grad

constexpr int kWgTile = 64;  // output tile: 64 rows (M) x 64 columns (K) per workgroup
constexpr int kWgStep = 32;  // voxels per MFMA step

struct PwWGeom {
  int K, M;
  uint32_t V;
  int splits;      // workgroups per sample along V
  uint32_t span;   // voxels per split (multiple of kWgStep)
  int kblocks;     // ceil(K / 64)
  int64_t stride;  // floats per partial slot: M * K + M
};

template <int PRO>
__global__ __launch_bounds__(kPwThreads) void pw_wgrad_kernel(const bf16_t* __restrict__ dy,
                                                              const bf16_t* __restrict__ x,
                                                              float* __restrict__ partial, PwWGeom g) {
  __shared__ float red[kWgTile * kWgTile + kWgTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int m0 = (blockIdx.y / g.kblocks) * kWgTile;
  const int k0 = (blockIdx.y % g.kblocks) * kWgTile;
  const int64_t n = blockIdx.z;
  const uint32_t V = g.V;
  const __amdgpu_buffer_rsrc_t dr = slab_rsrc(dy + n * g.M * static_cast<int64_t>(V), g.M * V * 2u);
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const uint32_t vbeg = blockIdx.x * g.span;
  const uint32_t vend = min(V, vbeg + g.span);

  bool mrow[4], krow[4];
  uint32_t mbase[4], kbase[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int m = m0 + 16 * t + c, k = k0 + 16 * t + c;
    mrow[t] = m < g.M;
    krow[t] = k < g.K;
    mbase[t] = static_cast<uint32_t>(m) * V * 2u;
    kbase[t] = static_cast<uint32_t>(k) * V * 2u;
  }
  const bool do_bias = k0 == 0;
  f32x4_t acc[4][4];
  float dbs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  auto load = [&](uint32_t v0, uint4 (&av)[4], uint4 (&bv)[4]) {
    const uint32_t vv = v0 + 8u * q;
    const bool ok = vv < vend;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      av[t] = buf_load16(dr, ok && mrow[t] ? mbase[t] + vv * 2u : kOob);
      bv[t] = buf_load16(xr, ok && krow[t] ? kbase[t] + vv * 2u : kOob);
    }
  };

  uint32_t v0 = vbeg + wave * kWgStep;
  uint4 an[4], bn[4];
  load(v0, an, bn);
  for (; v0 < vend; v0 += 4 * kWgStep) {
    uint4 av[4], bv[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      av[t] = an[t];
      bv[t] = bn[t];
    }
    if (v0 + 4 * kWgStep < vend) load(v0 + 4 * kWgStep, an, bn);
    if (PRO == MEDNEXT_PW_PROLOGUE_GELU) {
      // gelu(0) = 0, so out-of-range (zero) voxels stay zero.
#pragma unroll
      for (int t = 0; t < 4; ++t) bv[t] = gelu_vec(bv[t]);
    }
#pragma unroll
    for (int a = 0; a < 4; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b) acc[a][b] = mfma16x16x32(av[a], bv[b], acc[a][b]);
    if (do_bias) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint4 v = av[t];
        dbs[t] += (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) + (bf16_lo(v.z) + bf16_hi(v.z)) +
                  (bf16_lo(v.w) + bf16_hi(v.w));
      }
    }
  }

  // The four waves' tiles are summed into one LDS tile in wave order (every
  // lane owns the same elements in each wave, so turns only need barriers).
  float dbw[4];
  if (do_bias) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float s = dbs[t];
      s += __shfl_xor(s, 16);
      s += __shfl_xor(s, 32);
      dbw[t] = s;
    }
  }
  for (int turn = 0; turn < 4; ++turn) {
    if (wave == turn) {
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float& e = red[(16 * a + 4 * q + r) * kWgTile + 16 * b + c];
            e = turn == 0 ? acc[a][b][r] : e + acc[a][b][r];
          }
      if (do_bias && q == 0) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          float& e = red[kWgTile * kWgTile + 16 * t + c];
          e = turn == 0 ? dbw[t] : e + dbw[t];
        }
      }
    }
    __syncthreads();
  }
  float* out = partial + (n * gridDim.x + blockIdx.x) * g.stride;
  for (int e = threadIdx.x; e < kWgTile * kWgTile; e += kPwThreads) {
    const int m = m0 + e / kWgTile, k = k0 + e % kWgTile;
    if (m < g.M && k < g.K) out[static_cast<int64_t>(m) * g.K + k] = red[e];
  }
  if (do_bias && threadIdx.x < kWgTile) {
    const int m = m0 + threadIdx.x;
    if (m < g.M) out[static_cast<int64_t>(g.M) * g.K + m] = red[kWgTile * kWgTile + threadIdx.x];
  }
}

// dW / dB = fixed-order fp64 sum of the per-split partials. A block reduces
// kFinOut outputs; its kFinGroups thread groups each sum every kFinGroups-th
// slot, and the group sums are added in group order.
constexpr int kFinOut = 32;
constexpr int kFinGroups = 8;

__global__ __launch_bounds__(kFinOut* kFinGroups) void pw_wgrad_finish_kernel(
    const float* __restrict__ partial, bf16_t* __restrict__ dw, bf16_t* __restrict__ db, int64_t mk, int64_t m,
    int64_t slots, int64_t stride) {
  __shared__ double part[kFinGroups][kFinOut];
  const int lo = threadIdx.x % kFinOut, grp = threadIdx.x / kFinOut;
  const int64_t e = blockIdx.x * static_cast<int64_t>(kFinOut) + lo;
  const bool live = e < mk + m && (e < mk || db != nullptr);
  double s = 0.0;
  if (live) {
    for (int64_t t = grp; t < slots; t += kFinGroups) s += partial[t * stride + e];
  }
  part[grp][lo] = s;
  __syncthreads();
  if (grp == 0 && live) {
    double total = 0.0;
#pragma unroll
    for (int g = 0; g < kFinGroups; ++g) total += part[g][lo];
    const uint16_t v = f32_to_bf16(static_cast<float>(total));
    if (e < mk) {
      dw[e].bits = v;
    } else {
      db[e - mk].bits = v;
    }
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_pw_shape(int64_t n, int64_t k, int64_t m, int64_t v, int32_t dtype) {
  MEDNEXT_CHECK_ARG(dtype == MEDNEXT_DTYPE_BF16, "pointwise kernels take bfloat16 tensors");
  MEDNEXT_CHECK_ARG(n >= 1 && k >= 1 && m >= 1 && v >= 1, "empty pointwise problem");
  MEDNEXT_CHECK_ARG(k % 32 == 0, "input channels must be a multiple of 32");
  MEDNEXT_CHECK_ARG(m % 16 == 0, "output channels must be a multiple of 16");
  MEDNEXT_CHECK_ARG(v % 8 == 0, "voxels per sample must be a multiple of 8");
  MEDNEXT_CHECK_ARG(k * v * 2 < (int64_t{1} << 31) && m * v * 2 < (int64_t{1} << 31),
                    "one sample's tensor must be < 2 GiB");
  MEDNEXT_CHECK_ARG(n <= 65535, "batch too large");
  return MEDNEXT_STATUS_OK;
}

template <int PRO, int EPI>
void launch_fwd(dim3 grid, size_t lds, hipStream_t s, const bf16_t* x, const bf16_t* w, const bf16_t* b,
                const bf16_t* aux, bf16_t* y, const PwGeom& g) {
  hipLaunchKernelGGL((pw_fwd_kernel<PRO, EPI>), grid, dim3(kPwThreads), lds, s, x, w, b, aux, y, g);
}

}  // namespace
}  // namespace mednext

using namespace mednext;

extern "C" int32_t mednext_pointwise_fwd(const void* x, const void* weight, const void* bias, const void* aux,
                                         void* y, int64_t n, int64_t k, int64_t m, int64_t v,
                                         int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                         int32_t dtype, int32_t blocks_per_sample, void* stream) {
  if (int st = check_pw_shape(n, k, m, v, dtype)) return st;
  MEDNEXT_CHECK_ARG(x != nullptr && weight != nullptr && y != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG(k <= kMaxK, "input channels above 512 are not supported by the matrix-core GEMM");
  MEDNEXT_CHECK_ARG(weight_layout == 0 || weight_layout == 1, "weight_layout must be 0 ([M][K]) or 1 ([K][M])");
  MEDNEXT_CHECK_ARG(prologue == MEDNEXT_PW_PROLOGUE_NONE || prologue == MEDNEXT_PW_PROLOGUE_GELU, "bad prologue");
  MEDNEXT_CHECK_ARG(epilogue >= MEDNEXT_PW_EPILOGUE_BIAS && epilogue <= MEDNEXT_PW_EPILOGUE_GELU_GRAD, "bad epilogue");
  const bool needs_aux = epilogue == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL || epilogue == MEDNEXT_PW_EPILOGUE_GELU_GRAD;
  MEDNEXT_CHECK_ARG(!needs_aux || aux != nullptr, "this epilogue needs the aux tensor");
  MEDNEXT_CHECK_ARG(aligned16(x) && aligned16(weight) && aligned16(y) && (aux == nullptr || aligned16(aux)),
                    "pointwise tensors must be 16-byte aligned");
  MEDNEXT_CHECK_ARG(blocks_per_sample >= 1, "blocks_per_sample must be >= 1");
  PwGeom g;
  g.K = static_cast<int>(k);
  g.M = static_cast<int>(m);
  g.V = static_cast<uint32_t>(v);
  g.chunks = static_cast<int>(cdiv(v, kChunk));
  g.wt = weight_layout;
  const int bx = static_cast<int>(std::min<int64_t>(blocks_per_sample, cdiv(g.chunks, 4)));
  const dim3 grid(bx, static_cast<unsigned>(cdiv(m, kPwRows)), static_cast<unsigned>(n));
  const size_t lds = static_cast<size_t>(kPwRows) * k * 2;
  const auto s = static_cast<hipStream_t>(stream);
  const auto* xb = static_cast<const bf16_t*>(x);
  const auto* wb = static_cast<const bf16_t*>(weight);
  const auto* bb = static_cast<const bf16_t*>(bias);
  const auto* ab = static_cast<const bf16_t*>(aux);
  auto* yb = static_cast<bf16_t*>(y);
  if (prologue == MEDNEXT_PW_PROLOGUE_GELU) {
    switch (epilogue) {
      case MEDNEXT_PW_EPILOGUE_BIAS: launch_fwd<1, 0>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: launch_fwd<1, 1>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: launch_fwd<1, 2>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      default: launch_fwd<1, 3>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
    }
  } else {
    switch (epilogue) {
      case MEDNEXT_PW_EPILOGUE_BIAS: launch_fwd<0, 0>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: launch_fwd<0, 1>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: launch_fwd<0, 2>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
      default: launch_fwd<0, 3>(grid, lds, s, xb, wb, bb, ab, yb, g); break;
    }
  }
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

extern "C" size_t mednext_pointwise_wgrad_workspace_bytes(int64_t n, int64_t k, int64_t m, int64_t v,
                                                          int32_t splits) {
  if (n < 1 || k < 1 || m < 1 || v < 1 || splits < 1) return 0;
  return static_cast<size_t>(n) * splits * static_cast<size_t>(m * k + m) * sizeof(float);
}

extern "C" int32_t mednext_pointwise_wgrad(const void* grad_output, const void* x, void* grad_weight,
                                           void* grad_bias, void* workspace, size_t workspace_bytes,
                                           int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                           int32_t dtype, int32_t splits, void* stream) {
  if (int st = check_pw_shape(n, k, m, v, dtype)) return st;
  MEDNEXT_CHECK_ARG(grad_output != nullptr && x != nullptr && grad_weight != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG(prologue == MEDNEXT_PW_PROLOGUE_NONE || prologue == MEDNEXT_PW_PROLOGUE_GELU, "bad prologue");
  MEDNEXT_CHECK_ARG(splits >= 1 && splits <= 65535, "splits must be in [1, 65535]");
  MEDNEXT_CHECK_ARG(aligned16(grad_output) && aligned16(x), "pointwise tensors must be 16-byte aligned");
  const size_t need = mednext_pointwise_wgrad_workspace_bytes(n, k, m, v, splits);
  MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
  PwWGeom g;
  g.K = static_cast<int>(k);
  g.M = static_cast<int>(m);
  g.V = static_cast<uint32_t>(v);
  const int64_t steps = cdiv(v, kWgStep);
  const int64_t per_split = cdiv(steps, splits);
  g.span = static_cast<uint32_t>(per_split * kWgStep);
  g.splits = static_cast<int>(cdiv(v, static_cast<int64_t>(g.span)));
  g.kblocks = static_cast<int>(cdiv(k, kWgTile));
  g.stride = m * k + m;
  const dim3 grid(static_cast<unsigned>(g.splits), static_cast<unsigned>(cdiv(m, kWgTile) * g.kblocks),
                  static_cast<unsigned>(n));
  const auto s = static_cast<hipStream_t>(stream);
  auto* part = static_cast<float*>(workspace);
  if (prologue == MEDNEXT_PW_PROLOGUE_GELU) {
    hipLaunchKernelGGL((pw_wgrad_kernel<1>), grid, dim3(kPwThreads), 0, s, static_cast<const bf16_t*>(grad_output),
                       static_cast<const bf16_t*>(x), part, g);
  } else {
    hipLaunchKernelGGL((pw_wgrad_kernel<0>), grid, dim3(kPwThreads), 0, s, static_cast<const bf16_t*>(grad_output),
                       static_cast<const bf16_t*>(x), part, g);
  }
  MEDNEXT_CHECK_LAUNCH();
  const int64_t total = m * k + m;
  hipLaunchKernelGGL(pw_wgrad_finish_kernel, dim3(static_cast<unsigned>(cdiv(total, kFinOut))),
                     dim3(kFinOut * kFinGroups), 0, s,
                     part, static_cast<bf16_t*>(grad_weight), static_cast<bf16_t*>(grad_bias), m * k, m,
                     n * g.splits, g.stride);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}
