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
// GELU is the exact (erf) form (activation.h).
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "activation.h"
#include "cdna4.h"
#include "common.h"

namespace mednext {
namespace {

constexpr int kPwThreads = 256;  // 4 waves
constexpr int kChunk = 128;      // voxels per wave task (16 MFMA columns x 8 MFMAs)
constexpr int kMaxK = 2048;      // LDS weight block: 16 x 2048 bf16 = 64 KiB
constexpr int kMaxTiledK = 8192;  // the tiled product streams K in 32-channel slices
constexpr size_t kMaxWeightLds = 64 * 1024;
constexpr int kResidentWgs = 2 * 256;  // two 4-wave workgroups per CU fill the chip

struct PwGeom {
  int K, M;
  int ks;       // ceil(K / 32) slices of 32 channels
  uint32_t V;
  int chunks;   // ceil(V / kChunk)
  int mgroups;  // ceil(M / (16 * MT))
  int wgs;      // workgroups per (sample, row group)
  int wt;       // 1: weight stored [K][M] (A = W^T), 0: [M][K]
  int ksplit;   // tiled product: K ranges over workgroups (1: whole K, epilogue in the kernel)
  int kslices;  // tiled product: 32-channel slices per K range
};

__device__ inline uint32_t gelu_word(uint32_t w) {
  return pack_bf16x2(gelu_f(bf16_lo(w)), gelu_f(bf16_hi(w)));
}
__device__ inline uint4 gelu_vec(uint4 v) {
  return make_uint4(gelu_word(v.x), gelu_word(v.y), gelu_word(v.z), gelu_word(v.w));
}

// bf16(fma(x - c, s, t)) for the 8 values of one 16-byte group: c = 0 for an
// AFFINE record (x - 0 is x), the channel mean for a NORM record (the
// expression and fp32 operands mednext_group_norm_fwd rounds).
__device__ inline uint32_t affine_word(uint32_t w, float s, float t, float c) {
  return pack_bf16x2(fmaf(bf16_lo(w) - c, s, t), fmaf(bf16_hi(w) - c, s, t));
}
__device__ inline uint4 affine_vec(uint4 v, float s, float t, float c) {
  return make_uint4(affine_word(v.x, s, t, c), affine_word(v.y, s, t, c), affine_word(v.z, s, t, c),
                    affine_word(v.w, s, t, c));
}

// Extra operands of the AFFINE prologue and the ROW_REDUCE / AFFINE_SCALE /
// BIAS_GELU_PAIR epilogues (unused members are null).
struct PwExtra {
  const double* pcoef;  // [N][K][4]: (s, t, c, .) per (sample, input channel)
  int centred;          // NORM records: subtract c (entry 2) first; AFFINE: c = 0
  const double* ecoef;  // [N][M][2]: (c0, c1) per (sample, output row)
  double* rpart;        // [N][M][slots][2] row sums
  const bf16_t* aux2;   // AFFINE_SCALE: second per-element operand, shaped like y
  bf16_t* y2;           // BIAS_GELU_PAIR: second output, shaped like y
  int slots;
  float* kpart;         // tiled K-split: [ksplit][N][M][V rounded up to 8] fp32 partial products
};

constexpr bool epi_has_bias(int epi) {
  return epi == MEDNEXT_PW_EPILOGUE_BIAS || epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU ||
         epi == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL || epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR;
}

constexpr bool epi_has_aux(int epi) {
  return epi == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL || epi == MEDNEXT_PW_EPILOGUE_GELU_GRAD ||
         epi == MEDNEXT_PW_EPILOGUE_ROW_REDUCE || epi == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE ||
         epi == MEDNEXT_PW_EPILOGUE_AUX_SCALE;
}

// Per-row LDS vectors after the weight block: bias, then the AFFINE_SCALE
// coefficients c0 and c1 (16 MT floats each).
constexpr int kRowVecs = 3;

// The AFFINE / NORM prologue (a GRN or GroupNorm folded into the GEMM) is
// applied to each loaded X row, x -> bf16(fma(x - c[k], s[k], t[k])), with the
// per-channel (s, t, c) of the sample staged in LDS as floats (zero past K, so
// padded rows stay zero): bit for bit the value the unfolded normalisation
// would have stored. Used alike by the streaming, split-K and tiled forward
// kernels (the weight gradient applies the map to its reduced sums instead).
template <int PRO>
__device__ inline void prologue_rows(const uint4 (&r)[8], uint4 (&cur)[8], const float* kcoef, int k0) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if constexpr (PRO == MEDNEXT_PW_PROLOGUE_AFFINE) {
      const float* kc = kcoef + 3 * (k0 + i);
      cur[i] = affine_vec(r[i], kc[0], kc[1], kc[2]);
    } else {
      cur[i] = PRO == MEDNEXT_PW_PROLOGUE_GELU ? gelu_vec(r[i]) : r[i];
    }
  }
}

// Stages the sample's (s, t, c) of channels [0, kp) as floats (zero past K;
// c = 0 unless the records are centred).
__device__ inline void stage_affine(float* kcoef, const double* __restrict__ coef_n, int K, int kp, int centred) {
  for (int k = threadIdx.x; k < kp; k += kPwThreads) {
    const bool in = k < K;
    kcoef[3 * k] = in ? static_cast<float>(coef_n[k * 4]) : 0.f;
    kcoef[3 * k + 1] = in ? static_cast<float>(coef_n[k * 4 + 1]) : 0.f;
    kcoef[3 * k + 2] = in && centred ? static_cast<float>(coef_n[k * 4 + 2]) : 0.f;
  }
}

// X slice rows through the GELU prologue (the tiled kernel applies AFFINE
// with its own staged coefficients).
template <int PRO>
__device__ inline void apply_prologue(const uint4 (&r)[8], uint4 (&cur)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) cur[i] = PRO == MEDNEXT_PW_PROLOGUE_GELU ? gelu_vec(r[i]) : r[i];
}

__device__ inline float bf16_at(const uint4& v, int j) {
  const uint32_t wd = j / 2 == 0 ? v.x : j / 2 == 1 ? v.y : j / 2 == 2 ? v.z : v.w;
  return (j & 1) ? bf16_hi(wd) : bf16_lo(wd);
}

// One output row's 8 accumulators through a value epilogue (not ROW_REDUCE).
// `av` / `av2` hold the row's 8 aux / aux2 values (bf16), b the row bias,
// c0 / c1 the AFFINE_SCALE coefficients. BIAS_GELU_PAIR leaves GELU in v and
// GELU' in v2.
template <int EPI>
__device__ inline void epilogue_values(float (&v)[8], float (&v2)[8], const uint4& av, const uint4& av2, float b,
                                       float c0, float c1) {
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] += b;
  if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = gelu_f(v[j]);
  } else if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) {
#pragma unroll
    for (int j = 0; j < 8; ++j) gelu_pair(v[j], v[j], v2[j]);
  } else if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] += bf16_at(av, j);
  } else if constexpr (EPI == MEDNEXT_PW_EPILOGUE_GELU_GRAD) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= gelu_grad_f(bf16_at(av, j));
  } else if constexpr (EPI == MEDNEXT_PW_EPILOGUE_AUX_SCALE) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] *= bf16_at(av, j);
  } else if constexpr (EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = fmaf(v[j], c0, bf16_at(av, j) * c1) * bf16_at(av2, j);
  }
}

// ROW_REDUCE: add sum_j acc_j * aux_j and sum_j acc_j to (ra, rb).
__device__ inline void row_reduce_add(const float (&v)[8], const uint4& av, float& ra, float& rb) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    ra = fmaf(v[j], bf16_at(av, j), ra);
    rb += v[j];
  }
}

__device__ inline uint4 pack8(const float (&v)[8]) {
  return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                    pack_bf16x2(v[6], v[7]));
}

// Sum over the 16 lanes of a row group (lanes differing in bits 0-3), fixed order.
__device__ inline float sum16(float x) {
  x += __shfl_xor(x, 1);
  x += __shfl_xor(x, 2);
  x += __shfl_xor(x, 4);
  x += __shfl_xor(x, 8);
  return x;
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

// Eight consecutive bf16 of one row starting at byte `off`, of which only the
// first `nvalid` (< 8) exist: element loads, zeros for the rest. Used for the
// last, partial 8-voxel group of a row when V % 8 != 0, so no access reaches
// past the row.
__device__ inline uint4 load_partial(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t nvalid) {
  uint32_t wds[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (uint32_t e = 0; e < 8; ++e) {
    if (e < nvalid) {
      const uint32_t b = __builtin_amdgcn_raw_buffer_load_b16(r, off + 2u * e, 0, 0);
      wds[e / 2] |= b << (16u * (e & 1u));
    }
  }
  return make_uint4(wds[0], wds[1], wds[2], wds[3]);
}
__device__ inline void store_partial(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t nvalid, uint4 v) {
#pragma unroll
  for (uint32_t e = 0; e < 8; ++e) {
    if (e < nvalid) {
      const uint32_t wd = word(v, static_cast<int>(e / 2));
      __builtin_amdgcn_raw_buffer_store_b16(static_cast<unsigned short>(wd >> (16u * (e & 1u))), r, off + 2u * e,
                                            0, 0);
    }
  }
}

// One 8-voxel group of a row: a 16-byte load when all 8 voxels exist (the
// address is only 2-byte aligned when V % 8 != 0), element loads for the
// partial last group, zeros past the row (nvalid == 0 reads the out-of-range
// offset).
__device__ inline uint4 load_group(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t nvalid) {
  if (nvalid >= 8u) return buf_load16(r, off);
  if (nvalid == 0u) return buf_load16(r, kOob);
  return load_partial(r, off, nvalid);
}
__device__ inline void store_group(__amdgpu_buffer_rsrc_t r, uint32_t off, uint32_t nvalid, uint4 v) {
  if (nvalid >= 8u) {
    buf_store16(r, off, v);
  } else if (nvalid > 0u) {
    store_partial(r, off, nvalid, v);
  }
}

// Weight rows [m0, m0 + 16 MT) x [0, 32 KS) into LDS in A-fragment order
// (KS = ceil(K / 32)): fragment (ks, mt) is 64 lanes x 16 bytes at
// ((ks * MT + mt) * 64 + lane) * 16; entries outside [0, M) x [0, K) are zero.
// 16-byte global reads when whole 8-element groups exist, element reads
// otherwise (only for small, odd-shaped weights).
template <int MT>
__device__ void load_weight_block(const bf16_t* __restrict__ w, uint16_t* lds, const PwGeom& g, int m0) {
  constexpr int ROWS = 16 * MT;
  const int tid = threadIdx.x;
  const int kp = g.ks * 32;
  const uint16_t* __restrict__ wr = reinterpret_cast<const uint16_t*>(w);
  if (!g.wt) {  // w is [M][K]
    const bool vec = g.K % 8 == 0;
    const int per_row = kp / 8;
    for (int p = tid; p < ROWS * per_row; p += kPwThreads) {
      const int r = p / per_row, k8 = (p % per_row) * 8;
      const int m = m0 + r;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m < g.M && k8 < g.K) {
        const int64_t base = static_cast<int64_t>(m) * g.K + k8;
        if (vec) {
          v = *reinterpret_cast<const uint4*>(wr + base);
        } else {
          uint32_t wd[4] = {0u, 0u, 0u, 0u};
          for (int e = 0; e < 8 && k8 + e < g.K; ++e) wd[e / 2] |= static_cast<uint32_t>(wr[base + e]) << (16 * (e & 1));
          v = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        }
      }
      const int ks = k8 / 32, q = (k8 % 32) / 8, mt = r / 16, c = r % 16;
      *reinterpret_cast<uint4*>(lds + (((ks * MT + mt) * 64) + q * 16 + c) * 8) = v;
    }
  } else {  // w is [K][M]: A[m][k] = w[k][m]
    for (int p = tid; p < kp * ROWS; p += kPwThreads) {
      const int k = p / ROWS, r = p % ROWS;
      const int m = m0 + r;
      const uint16_t v = (k < g.K && m < g.M) ? wr[static_cast<int64_t>(k) * g.M + m] : uint16_t{0};
      const int ks = k / 32, q = (k % 32) / 8, i = k % 8, mt = r / 16, c = r % 16;
      lds[(((ks * MT + mt) * 64) + q * 16 + c) * 8 + i] = v;
    }
  }
}

// Forward / transposed product. Workgroup = one group of 16 MT output rows
// (its weight block in LDS) and a grid-stride run of 128-voxel chunks per
// wave. Per chunk a lane (q, n) loads X[32 ks + 8 q + i][v0 + 8 n + j]
// (i, j < 8: eight 16-byte loads per 32-channel slice), transposes the 8x8
// block in registers into the eight B operands, and multiplies every m-tile:
// C[16 mt + 4 q + r][n] of MFMA j is Y[m0 + 16 mt + 4 q + r][v0 + 8 n + j], so
// the epilogue stores 8 consecutive voxels (16 bytes) per row and lane.
//
// KS > 0: ceil(K / 32) = KS (1 to 4), the slice loop is unrolled and the first slice of the
// next chunk is loaded before this chunk's epilogue stores; with everything
// static the compiler's vmcnt waits then never wait for those stores (on CDNA
// the counter covers stores too). X slices rotate through two register
// buffers (KS odd alternates their roles per chunk). KS == 0: any K % 32 == 0
// with a runtime slice loop, prefetching one slice ahead inside a chunk.
// Channels at or past K read as zero (X rows and weight columns), rows at or
// past M are not stored, and a row's last partial 8-voxel group (V % 8 != 0)
// goes through element accesses, so any K <= 2048, M and V are accepted
// (larger K: the tiled product below).
template <int KS, int MT, int PRO, int EPI>
__global__ __launch_bounds__(kPwThreads, 2) void pw_fwd_kernel(const bf16_t* __restrict__ x,
                                                               const bf16_t* __restrict__ w,
                                                               const bf16_t* __restrict__ bias,
                                                               const bf16_t* __restrict__ aux,
                                                               bf16_t* __restrict__ y, PwGeom g, PwExtra ex) {
  constexpr bool kAux = epi_has_aux(EPI);
  constexpr bool kReduce = EPI == MEDNEXT_PW_EPILOGUE_ROW_REDUCE;
  extern __shared__ __align__(16) uint16_t pw_lds[];
  const int64_t lin = xcd_swizzle(blockIdx.x, gridDim.x);
  const int mg = static_cast<int>(lin % g.mgroups);
  const int64_t rest = lin / g.mgroups;
  const int bx = static_cast<int>(rest % g.wgs);
  const int64_t n = rest / g.wgs;
  const int m0 = mg * 16 * MT;
  constexpr bool kAffine = PRO == MEDNEXT_PW_PROLOGUE_AFFINE;
  load_weight_block<MT>(w, pw_lds, g, m0);
  // Row vectors of this row group as fp32 after the weight block (zero past
  // M): bias, then the AFFINE_SCALE coefficients c0, c1; then the AFFINE /
  // NORM prologue's (s, t, c) per input channel.
  float* const bias_lds = reinterpret_cast<float*>(pw_lds + static_cast<size_t>(16 * MT) * g.ks * 32);
  float* const c0_lds = bias_lds + 16 * MT;
  float* const c1_lds = c0_lds + 16 * MT;
  float* const kcoef = c1_lds + 16 * MT;
  if constexpr (kAffine) stage_affine(kcoef, ex.pcoef + n * g.K * 4, g.K, g.ks * 32, ex.centred);
  if (threadIdx.x < 16 * MT) {
    const int m = m0 + threadIdx.x;
    const bool in = m < g.M;
    const float b = (epi_has_bias(EPI) && bias != nullptr && in) ? bf16_to_f32(bias[m].bits) : 0.f;
    bias_lds[threadIdx.x] = b;
    if constexpr (EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE) {
      c0_lds[threadIdx.x] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2]) : 0.f;
      c1_lds[threadIdx.x] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2 + 1]) : 0.f;
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_col = lane & 15, q = lane >> 4;
  const uint32_t V = g.V;
  const int64_t yoff = n * g.M * static_cast<int64_t>(V);
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(y != nullptr ? y + yoff : x, y != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t y2r = slab_rsrc(ex.y2 != nullptr ? ex.y2 + yoff : x, ex.y2 != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t ar = slab_rsrc(aux != nullptr ? aux + yoff : x, aux != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t a2r =
      slab_rsrc(ex.aux2 != nullptr ? ex.aux2 + yoff : x, ex.aux2 != nullptr ? g.M * V * 2u : 0u);
  constexpr bool kAux2 = EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE;
  const int mtiles = min(MT, (g.M - m0 + 15) / 16);
  const uint4* frag = reinterpret_cast<const uint4*>(pw_lds) + lane;
  const int cstride = g.wgs * 4;
  auto valid = [&](int chunk) -> uint32_t {  // voxels of this lane's group that exist
    const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
    return (chunk < g.chunks && vl < V) ? min(8u, V - vl) : 0u;
  };
  auto load_slice = [&](int chunk, int ks, uint4 (&r)[8]) {
    const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
    const uint32_t nv = valid(chunk);
    const uint32_t row0 = 32u * ks + 8u * q;
    if (nv == 8u || nv == 0u) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool ok = nv != 0u && row0 + i < static_cast<uint32_t>(g.K);
        r[i] = buf_load16(xr, ok ? ((row0 + i) * V + vl) * 2u : kOob);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool ok = row0 + i < static_cast<uint32_t>(g.K);
        r[i] = load_group(xr, ((row0 + i) * V + vl) * 2u, ok ? nv : 0u);
      }
    }
  };
  auto mma_slice = [&](const uint4 (&r)[8], int ks, f32x4_t (&acc)[MT][8]) {
    uint4 cur[8];
    prologue_rows<PRO>(r, cur, kcoef, 32 * ks + 8 * q);
    uint4 bv[8];
    transpose8x8(cur, bv);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt < mtiles) {
        const uint4 a = frag[(ks * MT + mt) * 64];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[mt][j] = mfma16x16x32(a, bv[j], acc[mt][j]);
      }
    }
  };
  // aux rows, and for AFFINE_SCALE the aux2 rows in the upper half of av
  // (av[MT][4] for aux, av[MT][4 + r] for aux2 when MT == 1).
  auto load_aux = [&](int chunk, uint4 (&av)[MT][kAux2 ? 8 : 4]) {
    if constexpr (kAux) {
      const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
      const uint32_t nv = valid(chunk);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + 16 * mt + 4 * q + r;
          const uint32_t off = (static_cast<uint32_t>(min(m, g.M - 1)) * V + vl) * 2u;
          av[mt][r] = load_group(ar, off, m < g.M ? nv : 0u);
          if constexpr (kAux2) av[mt][4 + r] = load_group(a2r, off, m < g.M ? nv : 0u);
        }
    }
  };
  // ROW_REDUCE: this lane's running row sums (rows 16 mt + 4 q + r).
  float rsa[MT][4], rsb[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) rsa[mt][r] = rsb[mt][r] = 0.f;
  auto epilogue = [&](int chunk, const f32x4_t (&acc)[MT][8], const uint4 (&av)[MT][kAux2 ? 8 : 4]) {
    const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
    const uint32_t nv = valid(chunk);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt >= mtiles) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int mrow = m0 + 16 * mt + 4 * q + r;
        const uint32_t m = static_cast<uint32_t>(min(mrow, g.M - 1));
        const int lr = 16 * mt + 4 * q + r;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = acc[mt][j][r];
        if constexpr (kReduce) {
          // Voxels past V and rows past M have zero accumulators: no masking.
          row_reduce_add(v, av[mt][r], rsa[mt][r], rsb[mt][r]);
        } else {
          uint4 a4 = make_uint4(0u, 0u, 0u, 0u), b4 = a4;
          if constexpr (kAux) a4 = av[mt][r];
          if constexpr (kAux2) b4 = av[mt][4 + r];
          float v2[8];
          epilogue_values<EPI>(v, v2, a4, b4, bias_lds[lr], c0_lds[lr], c1_lds[lr]);
          const uint32_t nvr = mrow < g.M ? nv : 0u;
          store_group(yr, (m * V + vl) * 2u, nvr, pack8(v));
          if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) store_group(y2r, (m * V + vl) * 2u, nvr, pack8(v2));
        }
      }
    }
  };
  // ROW_REDUCE: one slot per wave (bx * 4 + wave), written once at the end
  // (zeros for a wave without chunks).
  auto flush_rows = [&]() {
    if constexpr (kReduce) {
      const int slot = bx * 4 + wave;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float a = sum16(rsa[mt][r]), b = sum16(rsb[mt][r]);
          const int mrow = m0 + 16 * mt + 4 * q + r;
          if (n_col == 0 && mrow < g.M) {
            double* dst = ex.rpart + ((n * g.M + mrow) * static_cast<int64_t>(ex.slots) + slot) * 2;
            dst[0] = a;
            dst[1] = b;
          }
        }
    }
  };

  int chunk = bx * 4 + wave;
  if (chunk >= g.chunks) {  // no barrier follows
    flush_rows();
    return;
  }
  if constexpr (KS > 0) {
    uint4 xb[2][8];
    load_slice(chunk, 0, xb[0]);
    // One chunk whose slice 0 sits in xb[P]; loads the next chunk's slice 0
    // into xb[(P + KS) % 2] before storing this chunk's outputs.
    auto process = [&](auto parity) {
      constexpr int P = decltype(parity)::value;
      constexpr int kAuxSlice = KS > 2 ? KS - 2 : 0;  // aux arrives during the last two slices
      uint4 av[MT][kAux2 ? 8 : 4];
      f32x4_t acc[MT][8];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ks == kAuxSlice) load_aux(chunk, av);
        if (ks + 1 < KS) {
          load_slice(chunk, ks + 1, xb[(P + ks + 1) % 2]);
        } else {
          load_slice(chunk + cstride, 0, xb[(P + KS) % 2]);
        }
        mma_slice(xb[(P + ks) % 2], ks, acc);
      }
      epilogue(chunk, acc, av);
      chunk += cstride;
    };
    for (;;) {
      process(std::integral_constant<int, 0>{});
      if (chunk >= g.chunks) break;
      if constexpr (KS % 2 == 1) {
        process(std::integral_constant<int, 1>{});
        if (chunk >= g.chunks) break;
      }
    }
    flush_rows();
  } else {
    const int ksteps = g.ks;
    for (; chunk < g.chunks; chunk += cstride) {
      uint4 av[MT][kAux2 ? 8 : 4];
      load_aux(chunk, av);
      f32x4_t acc[MT][8];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      uint4 xa[8], xn[8];
      load_slice(chunk, 0, xa);
      int ks = 0;
      for (; ks + 2 <= ksteps; ks += 2) {
        load_slice(chunk, ks + 1, xn);
        mma_slice(xa, ks, acc);
        if (ks + 2 < ksteps) load_slice(chunk, ks + 2, xa);
        mma_slice(xn, ks + 1, acc);
      }
      if (ks < ksteps) mma_slice(xa, ks, acc);
      epilogue(chunk, acc, av);
    }
    flush_rows();
  }
}

// Large-K forward (K >= 256: the stage 3-4 expansions and their input
// gradients, where V is small and a one-wave-per-chunk K loop would be a long
// serial chain). The workgroup takes one 128-voxel chunk at a time and its
// four waves split the 32-channel slices (wave w: slices w, w + 4, ...). The
// partial accumulators are summed through LDS in wave order (fixed, so the
// result is reproducible) and wave w then finishes rows 4 q + w of every
// m-tile.
template <int MT, int PRO, int EPI>
__global__ __launch_bounds__(kPwThreads, 2) void pw_fwd_splitk_kernel(const bf16_t* __restrict__ x,
                                                                      const bf16_t* __restrict__ w,
                                                                      const bf16_t* __restrict__ bias,
                                                                      const bf16_t* __restrict__ aux,
                                                                      bf16_t* __restrict__ y, PwGeom g, PwExtra ex) {
  constexpr bool kAux = epi_has_aux(EPI);
  constexpr bool kReduce = EPI == MEDNEXT_PW_EPILOGUE_ROW_REDUCE;
  extern __shared__ __align__(16) uint16_t pw_lds[];
  const int64_t lin = xcd_swizzle(blockIdx.x, gridDim.x);
  const int mg = static_cast<int>(lin % g.mgroups);
  const int64_t rest = lin / g.mgroups;
  const int bx = static_cast<int>(rest % g.wgs);
  const int64_t n = rest / g.wgs;
  const int m0 = mg * 16 * MT;
  constexpr bool kAffine = PRO == MEDNEXT_PW_PROLOGUE_AFFINE;
  load_weight_block<MT>(w, pw_lds, g, m0);
  float* const bias_lds = reinterpret_cast<float*>(pw_lds + static_cast<size_t>(16 * MT) * g.ks * 32);
  float* const c0_lds = bias_lds + 16 * MT;
  float* const c1_lds = c0_lds + 16 * MT;
  float* const red = bias_lds + kRowVecs * 16 * MT;  // [MT][8][4][64] partial sums
  float* const kcoef = red + MT * 8 * 4 * 64;        // AFFINE / NORM: (s, t, c) per input channel
  if constexpr (kAffine) stage_affine(kcoef, ex.pcoef + n * g.K * 4, g.K, g.ks * 32, ex.centred);
  if (threadIdx.x < 16 * MT) {
    const int m = m0 + threadIdx.x;
    const bool in = m < g.M;
    const float b = (epi_has_bias(EPI) && bias != nullptr && in) ? bf16_to_f32(bias[m].bits) : 0.f;
    bias_lds[threadIdx.x] = b;
    if constexpr (EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE) {
      c0_lds[threadIdx.x] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2]) : 0.f;
      c1_lds[threadIdx.x] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2 + 1]) : 0.f;
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_col = lane & 15, q = lane >> 4;
  const uint32_t V = g.V;
  const int64_t yoff = n * g.M * static_cast<int64_t>(V);
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(y != nullptr ? y + yoff : x, y != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t y2r = slab_rsrc(ex.y2 != nullptr ? ex.y2 + yoff : x, ex.y2 != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t ar = slab_rsrc(aux != nullptr ? aux + yoff : x, aux != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t a2r =
      slab_rsrc(ex.aux2 != nullptr ? ex.aux2 + yoff : x, ex.aux2 != nullptr ? g.M * V * 2u : 0u);
  constexpr bool kAux2 = EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE;
  const int mtiles = min(MT, (g.M - m0 + 15) / 16);
  const uint4* frag = reinterpret_cast<const uint4*>(pw_lds) + lane;
  float rsa[MT], rsb[MT];  // ROW_REDUCE running sums of rows 16 mt + 4 q + wave
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) rsa[mt] = rsb[mt] = 0.f;

  for (int chunk = bx; chunk < g.chunks; chunk += g.wgs) {
    const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
    const uint32_t nv = vl < V ? min(8u, V - vl) : 0u;
    auto load_slice = [&](int ks, uint4 (&r)[8]) {
      const uint32_t row0 = 32u * ks + 8u * q;
      const bool in = ks < g.ks;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const bool ok = in && row0 + i < static_cast<uint32_t>(g.K);
        if (nv == 8u || nv == 0u) {
          r[i] = buf_load16(xr, ok && nv != 0u ? ((row0 + i) * V + vl) * 2u : kOob);
        } else {
          r[i] = load_group(xr, ((row0 + i) * V + vl) * 2u, ok ? nv : 0u);
        }
      }
    };
    uint4 av[MT], av2[MT];
    if constexpr (kAux) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = m0 + 16 * mt + 4 * q + wave;
        const uint32_t off = (static_cast<uint32_t>(min(m, g.M - 1)) * V + vl) * 2u;
        av[mt] = load_group(ar, off, m < g.M ? nv : 0u);
        if constexpr (kAux2) av2[mt] = load_group(a2r, off, m < g.M ? nv : 0u);
      }
    }
    f32x4_t acc[MT][8];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto mma_slice = [&](const uint4 (&r)[8], int ks) {
      uint4 cur[8];
      prologue_rows<PRO>(r, cur, kcoef, 32 * ks + 8 * q);
      uint4 bv[8];
      transpose8x8(cur, bv);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (mt < mtiles) {
          const uint4 a = frag[(ks * MT + mt) * 64];
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[mt][j] = mfma16x16x32(a, bv[j], acc[mt][j]);
        }
      }
    };
    uint4 xa[8], xn[8];
    int ks = wave;
    load_slice(ks, xa);
    for (; ks + 4 < g.ks; ks += 8) {
      load_slice(ks + 4, xn);
      mma_slice(xa, ks);
      load_slice(ks + 8, xa);
      mma_slice(xn, ks + 4);
    }
    if (ks < g.ks) mma_slice(xa, ks);

#pragma unroll
    for (int turn = 0; turn < 4; ++turn) {
      if (wave == turn) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              float& e = red[((mt * 8 + j) * 4 + r) * 64 + lane];
              e = turn == 0 ? acc[mt][j][r] : e + acc[mt][j][r];
            }
      }
      __syncthreads();
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (mt >= mtiles) continue;
      const int mrow = m0 + 16 * mt + 4 * q + wave;
      const uint32_t m = static_cast<uint32_t>(min(mrow, g.M - 1));
      const int lr = 16 * mt + 4 * q + wave;
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = red[((mt * 8 + j) * 4 + wave) * 64 + lane];
      if constexpr (kReduce) {
        row_reduce_add(v, av[mt], rsa[mt], rsb[mt]);
      } else {
        uint4 a4 = make_uint4(0u, 0u, 0u, 0u), b4 = a4;
        if constexpr (kAux) a4 = av[mt];
        if constexpr (kAux2) b4 = av2[mt];
        float v2[8];
        epilogue_values<EPI>(v, v2, a4, b4, bias_lds[lr], c0_lds[lr], c1_lds[lr]);
        const uint32_t nvr = mrow < g.M ? nv : 0u;
        store_group(yr, (m * V + vl) * 2u, nvr, pack8(v));
        if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) store_group(y2r, (m * V + vl) * 2u, nvr, pack8(v2));
      }
    }
    __syncthreads();  // the next chunk's turn 0 overwrites the sums read above
  }
  if constexpr (kReduce) {
    // One slot per workgroup (bx); zeros when it had no chunk.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const float a = sum16(rsa[mt]), b = sum16(rsb[mt]);
      const int mrow = m0 + 16 * mt + 4 * q + wave;
      if (n_col == 0 && mrow < g.M) {
        double* dst = ex.rpart + ((n * g.M + mrow) * static_cast<int64_t>(ex.slots) + bx) * 2;
        dst[0] = a;
        dst[1] = b;
      }
    }
  }
}

// ------------------------------------------------------------- tiled product
//
// The kernels above keep X out of LDS, so a workgroup of 16 MT output rows
// reads its X columns once per row group: at wide M (the GRN input gradients,
// M = 4C) or deep K (the project GEMMs of the wide expansions) X is read
// M / (16 MT) times. The tiled kernel shares each X tile across 64 MT output
// rows instead. Workgroup = rows [m0, m0 + 64 MT) x one 128-voxel chunk; wave w
// owns rows m0 + 16 MT w .. + 16 MT. K advances in steps of two 32-channel
// slices through a double-buffered LDS stage:
//   waves 0, 1  load X slice 2 s + w (eight 16-byte loads per lane, as in
//               pw_fwd_kernel), apply the prologue, transpose in registers and
//               store the eight B operands (the whole workgroup's for that
//               slice) to LDS;
//   waves 2, 3  load weight slice 2 s + w - 2 for all 64 MT rows into LDS in
//               A-fragment order ([K][M] weights through the same 8x8 register
//               transpose);
//   all waves   one barrier, then MT x 8 MFMAs per slice from LDS.
// The next step's loads are issued before the MFMAs of this one. The AFFINE
// prologue is applied to X (bf16(x s + t) per channel, coefficients staged in
// LDS), so no per-launch weight folding is needed. Requirements (checked by
// the host): K % 32 == 0, M % 16 == 0, no ROW_REDUCE epilogue.
//
// K split over workgroups (g.ksplit > 1, the deep products whose tiles alone
// leave the chip short of workgroups): workgroup (tile, r) multiplies only the
// slices [r * kslices, (r + 1) * kslices) and stores its fp32 tile to
// ex.kpart; pw_ksplit_epilogue_kernel then adds the K ranges in range order
// (deterministic) and applies the epilogue.
constexpr int kTileSlices = 2;

template <int MT, int PRO, int EPI>
__global__ __launch_bounds__(kPwThreads, 2) void pw_fwd_tiled_kernel(const bf16_t* __restrict__ x,
                                                                     const bf16_t* __restrict__ w,
                                                                     const bf16_t* __restrict__ bias,
                                                                     const bf16_t* __restrict__ aux,
                                                                     bf16_t* __restrict__ y, PwGeom g, PwExtra ex) {
  static_assert(MT == 1 || MT == 2, "tiled product: 64 or 128 rows per workgroup");
  static_assert(EPI != MEDNEXT_PW_EPILOGUE_ROW_REDUCE, "ROW_REDUCE runs the streaming kernels");
  constexpr int BM = 64 * MT;
  constexpr int F16 = 4 * MT;  // 16-row fragments per workgroup
  constexpr int XS = 8 * 64;   // uint4 per X slice: eight B operands x 64 lanes
  constexpr int WS = F16 * 64; // uint4 per weight slice
  constexpr int SLICE = XS + WS;  // one slice's B operands followed by its A fragments
  constexpr bool kAux = epi_has_aux(EPI);
  constexpr bool kAux2 = EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE;
  constexpr bool kAffine = PRO == MEDNEXT_PW_PROLOGUE_AFFINE;
  extern __shared__ __align__(16) uint16_t pw_lds[];
  uint4* const stages = reinterpret_cast<uint4*>(pw_lds);
  // This workgroup's K range: slices [kbase, kbase + nks).
  int64_t lin = xcd_swizzle(blockIdx.x, gridDim.x);
  const int ksp = static_cast<int>(lin % g.ksplit);
  lin /= g.ksplit;
  const int kbase = ksp * g.kslices;
  const int nks = min(g.kslices, g.ks - kbase);
  // LDS holds only the slices used: min(2, nks) per stage, and a second stage
  // only when the range takes more than one step.
  const int sps = min(kTileSlices, nks);
  const int nstages = nks > kTileSlices ? 2 : 1;
  float* const bias_lds = reinterpret_cast<float*>(stages + nstages * sps * SLICE);
  float* const c0_lds = bias_lds + BM;
  float* const c1_lds = c0_lds + BM;
  float* const kcoef = c1_lds + BM;  // AFFINE / NORM: (s, t, c) per input channel

  const int mg = static_cast<int>(lin % g.mgroups);
  const int64_t rest = lin / g.mgroups;
  const int chunk = static_cast<int>(rest % g.chunks);
  const int64_t n = rest / g.chunks;
  const int m0 = mg * BM;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n_col = lane & 15, q = lane >> 4;
  const bool split = g.ksplit > 1;

  for (int r = threadIdx.x; r < BM; r += kPwThreads) {
    const int m = m0 + r;
    const bool in = m < g.M;
    bias_lds[r] = (epi_has_bias(EPI) && bias != nullptr && in) ? bf16_to_f32(bias[m].bits) : 0.f;
    if constexpr (kAux2) {
      c0_lds[r] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2]) : 0.f;
      c1_lds[r] = in ? static_cast<float>(ex.ecoef[(n * g.M + m) * 2 + 1]) : 0.f;
    }
  }
  if constexpr (kAffine) stage_affine(kcoef, ex.pcoef + n * g.K * 4, g.K, g.K, ex.centred);

  const uint32_t V = g.V;
  const uint32_t vl = static_cast<uint32_t>(chunk) * kChunk + 8u * n_col;
  const uint32_t nv = vl < V ? min(8u, V - vl) : 0u;
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const __amdgpu_buffer_rsrc_t wr = slab_rsrc(w, static_cast<uint32_t>(g.M) * g.K * 2u);
  const bool loads_x = wave < kTileSlices;
  // Weight loaders: [M][K] -> lane = (q, row in fragment), one 16-byte load per
  // fragment; [K][M] -> lane = (q, 8-row octet), eight row loads + transpose.
  const int wslot = wave - kTileSlices;
  constexpr int kOctets = BM / 8;  // 8-row octets of the workgroup
  constexpr int kPairs = 4 * kOctets;  // (q, octet) pairs, <= 64
  const int oct = lane >> 2, oq = lane & 3;

  uint4 rg[8];  // the loads of one slice (X rows or weight fragments)
  auto load_slice = [&](int local) {
    const int slice = kbase + local;
    if (loads_x) {
      const uint32_t row0 = 32u * slice + 8u * q;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t off = ((row0 + i) * V + vl) * 2u;
        rg[i] = (nv == 8u || nv == 0u) ? buf_load16(xr, nv != 0u ? off : kOob) : load_group(xr, off, nv);
      }
    } else if (!g.wt) {
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const uint32_t m = static_cast<uint32_t>(m0 + 16 * f + n_col);
        const uint32_t off = (m * static_cast<uint32_t>(g.K) + 32u * slice + 8u * q) * 2u;
        rg[f] = (f < F16 && m < static_cast<uint32_t>(g.M)) ? buf_load16(wr, off) : make_uint4(0u, 0u, 0u, 0u);
      }
    } else {
      const int m = m0 + 8 * oct;
      const bool ok = lane < kPairs && m < g.M;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t k = 32u * slice + 8u * oq + e;
        rg[e] = ok ? buf_load16(wr, (k * static_cast<uint32_t>(g.M) + m) * 2u) : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  };
  auto store_slice = [&](int local, uint4* stage) {
    const int slice = kbase + local;
    if (loads_x) {
      uint4 cur[8];
      if constexpr (kAffine) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float* kc = kcoef + 3 * (32 * slice + 8 * q + i);
          cur[i] = affine_vec(rg[i], kc[0], kc[1], kc[2]);
        }
      } else {
        apply_prologue<PRO>(rg, cur);
      }
      uint4 bv[8];
      transpose8x8(cur, bv);
      uint4* dst = stage + wave * SLICE + lane;
#pragma unroll
      for (int j = 0; j < 8; ++j) dst[j * 64] = bv[j];
    } else {
      uint4* dst = stage + wslot * SLICE + XS;
      if (!g.wt) {
#pragma unroll
        for (int f = 0; f < F16; ++f) dst[f * 64 + lane] = rg[f];
      } else if (lane < kPairs) {
        uint4 bv[8];
        transpose8x8(rg, bv);  // bv[c] = 8 channels of row m0 + 8 oct + c
        uint4* frag = dst + (oct >> 1) * 64 + oq * 16 + 8 * (oct & 1);
#pragma unroll
        for (int c = 0; c < 8; ++c) frag[c] = bv[c];
      }
    }
  };

  f32x4_t acc[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[mt][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const bool rows_live = m0 + 16 * MT * wave < g.M;
  // The epilogue's per-element operands are loaded before the K loop, so
  // their latency hides behind it (zeros for tiles past M).
  const int64_t yoff = n * g.M * static_cast<int64_t>(V);
  const __amdgpu_buffer_rsrc_t ar = slab_rsrc(aux != nullptr ? aux + yoff : y, aux != nullptr ? g.M * V * 2u : 0u);
  const __amdgpu_buffer_rsrc_t a2r =
      slab_rsrc(ex.aux2 != nullptr ? ex.aux2 + yoff : y, ex.aux2 != nullptr ? g.M * V * 2u : 0u);
  uint4 av[MT][4], av2[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const bool live = m0 + 16 * MT * wave + 16 * mt < g.M;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      av[mt][r] = av2[mt][r] = make_uint4(0u, 0u, 0u, 0u);
      const uint32_t off = (static_cast<uint32_t>(m0 + 16 * MT * wave + 16 * mt + 4 * q + r) * V + vl) * 2u;
      const uint32_t nload = live && !split ? nv : 0u;  // K-split: the epilogue kernel reads them
      if constexpr (kAux) av[mt][r] = load_group(ar, off, nload);
      if constexpr (kAux2) av2[mt][r] = load_group(a2r, off, nload);
    }
  }
  const int steps = (nks + kTileSlices - 1) / kTileSlices;
  const int my_slice = loads_x ? wave : wslot;
  if (my_slice < nks) load_slice(my_slice);
  __syncthreads();  // row vectors and AFFINE coefficients
  for (int s = 0; s < steps; ++s) {
    uint4* const stage = stages + (s & 1) * sps * SLICE;
    const int slice = kTileSlices * s + my_slice;
    if (slice < nks) store_slice(slice, stage);
    if (slice + kTileSlices < nks) load_slice(slice + kTileSlices);
    __syncthreads();
    if (rows_live) {
#pragma unroll
      for (int sl = 0; sl < kTileSlices; ++sl) {
        if (kTileSlices * s + sl < nks) {
          const uint4* xs = stage + sl * SLICE + lane;
          const uint4* ws = stage + sl * SLICE + XS + (MT * wave) * 64 + lane;
          uint4 a[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) a[mt] = ws[mt * 64];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const uint4 b = xs[j * 64];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt][j] = mfma16x16x32(a[mt], b, acc[mt][j]);
          }
        }
      }
    }
  }
  if (!rows_live) return;

  if (split) {
    // fp32 tile of this K range: kpart[n][ksp][m][8 * ceil(V / 8)], 8 voxels per row and lane.
    const int64_t vp = static_cast<int64_t>((V + 7u) & ~7u);
    float* __restrict__ part = ex.kpart + (n * g.ksplit + ksp) * g.M * vp;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (m0 + 16 * MT * wave + 16 * mt >= g.M || nv == 0u) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + 16 * MT * wave + 16 * mt + 4 * q + r;
        float4* dst = reinterpret_cast<float4*>(part + m * vp + vl);
        dst[0] = make_float4(acc[mt][0][r], acc[mt][1][r], acc[mt][2][r], acc[mt][3][r]);
        dst[1] = make_float4(acc[mt][4][r], acc[mt][5][r], acc[mt][6][r], acc[mt][7][r]);
      }
    }
    return;
  }

  const __amdgpu_buffer_rsrc_t yr = slab_rsrc(y + yoff, g.M * V * 2u);
  const __amdgpu_buffer_rsrc_t y2r = slab_rsrc(ex.y2 != nullptr ? ex.y2 + yoff : y, ex.y2 != nullptr ? g.M * V * 2u : 0u);
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int lr0 = 16 * MT * wave + 16 * mt + 4 * q;
    if (m0 + 16 * MT * wave + 16 * mt >= g.M) continue;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int lr = lr0 + r;
      float v[8], v2[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = acc[mt][j][r];
      epilogue_values<EPI>(v, v2, av[mt][r], av2[mt][r], bias_lds[lr], c0_lds[lr], c1_lds[lr]);
      const uint32_t off = (static_cast<uint32_t>(m0 + lr) * V + vl) * 2u;
      store_group(yr, off, nv, pack8(v));
      if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) store_group(y2r, off, nv, pack8(v2));
    }
  }
}

// Epilogue of the K-split tiled product: per thread one row's 8 consecutive
// voxels, the K ranges' fp32 partials added in range order, then the same
// value epilogue as the fused kernels (bias, GELU, residual, GELU', scales).
template <int EPI>
__global__ __launch_bounds__(kPwThreads) void pw_ksplit_epilogue_kernel(const bf16_t* __restrict__ bias,
                                                                        const bf16_t* __restrict__ aux,
                                                                        bf16_t* __restrict__ y, PwGeom g,
                                                                        PwExtra ex, int64_t n_samples) {
  const uint32_t V = g.V;
  const uint32_t groups = (V + 7u) / 8u;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kPwThreads + threadIdx.x;
  if (t >= n_samples * g.M * groups) return;
  const int64_t row = t / groups;  // n * M + m
  const uint32_t gi = static_cast<uint32_t>(t - row * groups);
  const int64_t n = row / g.M;
  const int m = static_cast<int>(row - n * g.M);
  const int64_t vp = static_cast<int64_t>(groups) * 8;
  const float* __restrict__ p = ex.kpart + ((n * g.ksplit) * g.M + m) * vp + 8 * gi;
  float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, v2[8];
  for (int r = 0; r < g.ksplit; ++r) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] += a.x; v[1] += a.y; v[2] += a.z; v[3] += a.w;
    v[4] += b.x; v[5] += b.y; v[6] += b.z; v[7] += b.w;
    p += g.M * vp;
  }
  const uint32_t vl = 8u * gi;
  const uint32_t nv = min(8u, V - vl);
  const int64_t yoff = n * g.M * static_cast<int64_t>(V);
  const uint32_t off = (static_cast<uint32_t>(m) * V + vl) * 2u;
  uint4 av = make_uint4(0u, 0u, 0u, 0u), av2 = av;
  if constexpr (epi_has_aux(EPI)) av = load_group(slab_rsrc(aux + yoff, g.M * V * 2u), off, nv);
  float c0 = 0.f, c1 = 0.f;
  if constexpr (EPI == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE) {
    av2 = load_group(slab_rsrc(ex.aux2 + yoff, g.M * V * 2u), off, nv);
    c0 = static_cast<float>(ex.ecoef[row * 2]);
    c1 = static_cast<float>(ex.ecoef[row * 2 + 1]);
  }
  const float b = (epi_has_bias(EPI) && bias != nullptr) ? bf16_to_f32(bias[m].bits) : 0.f;
  epilogue_values<EPI>(v, v2, av, av2, b, c0, c1);
  store_group(slab_rsrc(y + yoff, g.M * V * 2u), off, nv, pack8(v));
  if constexpr (EPI == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) {
    store_group(slab_rsrc(ex.y2 + yoff, g.M * V * 2u), off, nv, pack8(v2));
  }
}

// ---------------------------------------------------------------- weight grad

constexpr int kWgStage = 128;   // voxels per LDS stage (4 waves x one 32-voxel MFMA step)
constexpr int kWgPitch = kWgStage + 8;  // LDS row pitch (elements): 272 bytes

struct PwWGeom {
  int K, M;
  uint32_t V;
  int splits;      // workgroups per sample along V
  uint32_t span;   // voxels per split (multiple of kWgStage)
  int mblocks, kblocks;
  int64_t stride;  // floats per partial slot: M * K + M
};

// dW[M][K] = sum_v dY[M][v] X[K][v] over one split's voxel range, for an output
// tile of 16 TM rows x 16 TK columns. Per 128-voxel stage the workgroup copies
// the tile's dY rows and X rows into LDS with row-contiguous 16-byte loads (16
// lanes cover 256 bytes of one row; GELU applied to X on the way when the
// prologue asks for it), and wave w multiplies voxels 32 w .. 32 w + 31 of the
// stage: A = 8 consecutive voxels of a dY row, B = the same voxels of an X row
// per lane. The next stage's loads are in flight during the MFMAs. dB[m] =
// sum_v dY[m][v] comes from the same loads: every thread owns fixed rows.
template <int TM, int TK, int PRO>
__global__ __launch_bounds__(kPwThreads, TM * TK >= 16 ? 3 : 4) void pw_wgrad_kernel(const bf16_t* __restrict__ dy,
                                                                 const bf16_t* __restrict__ x,
                                                                 float* __restrict__ partial, PwWGeom g) {
  constexpr int RM = 16 * TM, RK = 16 * TK, ROWS = RM + RK;
  constexpr int NLD = ROWS * (kWgStage / 8) / kPwThreads;  // 16-byte loads per thread per stage
  static_assert(NLD * kPwThreads == ROWS * (kWgStage / 8), "rows must fill the workgroup");
  constexpr int TILE = ROWS * kWgPitch;                     // elements
  constexpr int RED = RM * RK + RM;                          // floats for the final reduction
  constexpr int SMEM = (TILE * 2 > RED * 4 ? TILE * 2 : RED * 4);
  __shared__ __align__(16) unsigned char smem[SMEM];
  uint16_t* const tile = reinterpret_cast<uint16_t*>(smem);
  float* const red = reinterpret_cast<float*>(smem);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int64_t lin = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tl = static_cast<int>(lin % (g.mblocks * g.kblocks));
  const int64_t rest = lin / (g.mblocks * g.kblocks);
  const int split = static_cast<int>(rest % g.splits);
  const int64_t n = rest / g.splits;
  const int m0 = (tl / g.kblocks) * RM;
  const int k0 = (tl % g.kblocks) * RK;
  const uint32_t V = g.V;
  const __amdgpu_buffer_rsrc_t dr = slab_rsrc(dy + n * g.M * static_cast<int64_t>(V), g.M * V * 2u);
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const uint32_t vbeg = static_cast<uint32_t>(split) * g.span;
  const uint32_t vend = min(V, vbeg + g.span);
  const bool do_bias = k0 == 0;

  // Load slot u of this thread: tile row r = tid / 16 + 16 u (dY rows first,
  // then X rows), voxels 8 (tid % 16) .. + 7 of the stage.
  const int grp = threadIdx.x & 15;
  uint32_t rbase[NLD];
  bool rok[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = (threadIdx.x >> 4) + 16 * u;
    const int row = r < RM ? m0 + r : k0 + (r - RM);
    rok[u] = r < RM ? row < g.M : row < g.K;
    rbase[u] = static_cast<uint32_t>(rok[u] ? row : 0) * V * 2u;
  }
  auto load = [&](uint32_t v, uint4 (&regs)[NLD]) {
    const uint32_t vv = v + 8u * grp;
    const uint32_t nv = vv < vend ? min(8u, vend - vv) : 0u;
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int r = (threadIdx.x >> 4) + 16 * u;
      const __amdgpu_buffer_rsrc_t rs = r < RM ? dr : xr;
      if (nv == 8u || nv == 0u) {
        regs[u] = buf_load16(rs, nv != 0u && rok[u] ? rbase[u] + vv * 2u : kOob);
      } else {
        regs[u] = load_group(rs, rbase[u] + vv * 2u, rok[u] ? nv : 0u);
      }
    }
  };
  float dbs[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) dbs[u] = 0.f;
  auto stash = [&](const uint4 (&regs)[NLD]) {
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int r = (threadIdx.x >> 4) + 16 * u;
      uint4 v = regs[u];
      if (r < RM) {
        if (do_bias) {
          dbs[u] += (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) +
                    (bf16_lo(v.z) + bf16_hi(v.z)) + (bf16_lo(v.w) + bf16_hi(v.w));
        }
      } else if (PRO == MEDNEXT_PW_PROLOGUE_GELU) {
        v = gelu_vec(v);  // gelu(0) = 0: missing voxels stay zero
      }
      *reinterpret_cast<uint4*>(tile + r * kWgPitch + 8 * grp) = v;
    }
  };

  f32x4_t acc[TM][TK];
#pragma unroll
  for (int a = 0; a < TM; ++a)
#pragma unroll
    for (int b = 0; b < TK; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 regs[NLD];
  uint32_t v = vbeg;
  load(v, regs);
  while (v < vend) {
    stash(regs);
    __syncthreads();
    load(v + kWgStage, regs);  // next stage in flight during the MFMAs
    uint4 bf[TK];
#pragma unroll
    for (int b = 0; b < TK; ++b)
      bf[b] = *reinterpret_cast<const uint4*>(tile + (RM + 16 * b + c) * kWgPitch + 32 * wave + 8 * q);
#pragma unroll
    for (int a = 0; a < TM; ++a) {
      const uint4 af = *reinterpret_cast<const uint4*>(tile + (16 * a + c) * kWgPitch + 32 * wave + 8 * q);
#pragma unroll
      for (int b = 0; b < TK; ++b) acc[a][b] = mfma16x16x32(af, bf[b], acc[a][b]);
    }
    __syncthreads();
    v += kWgStage;
  }

  // The four waves' tiles are summed into one LDS tile in wave order (every
  // lane owns the same elements in each wave, so turns only need barriers).
  for (int turn = 0; turn < 4; ++turn) {
    if (wave == turn) {
#pragma unroll
      for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int b = 0; b < TK; ++b)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float& e = red[(16 * a + 4 * q + r) * RK + 16 * b + c];
            e = turn == 0 ? acc[a][b][r] : e + acc[a][b][r];
          }
    }
    __syncthreads();
  }
  if (do_bias) {
    // Row sums: the 16 threads of a row are 16 consecutive lanes of one wave.
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      float sum = dbs[u];
      sum += __shfl_xor(sum, 1);
      sum += __shfl_xor(sum, 2);
      sum += __shfl_xor(sum, 4);
      sum += __shfl_xor(sum, 8);
      const int r = (threadIdx.x >> 4) + 16 * u;
      if (grp == 0 && r < RM) red[RM * RK + r] = sum;
    }
    __syncthreads();
  }
  float* out = partial + (n * g.splits + split) * g.stride;
  for (int e = threadIdx.x; e < RM * RK; e += kPwThreads) {
    const int m = m0 + e / RK, k = k0 + e % RK;
    if (m < g.M && k < g.K) out[static_cast<int64_t>(m) * g.K + k] = red[e];
  }
  if (do_bias && threadIdx.x < RM) {
    const int m = m0 + threadIdx.x;
    if (m < g.M) out[static_cast<int64_t>(g.M) * g.K + m] = red[RM * RK + threadIdx.x];
  }
}

// Wide weight-gradient tile: 128 dW rows x 128 columns per workgroup, so X is
// read once per 128 rows of M and dY once per 128 columns of K (the 64 x 64
// kernel above reads them twice as often; at the MedNeXt v2 hidden widths
// that is 3-7x the algorithmic traffic). Per 128-voxel stage the 256 tile rows
// (128 dY, 128 X) go through LDS exactly as above, but the waves split the
// output instead of the voxels: wave w owns the 64 x 64 quadrant
// (w / 2, w % 2) and runs 4 x 4 MFMA tiles over all four 32-voxel steps of the
// stage. No cross-wave reduction is needed; each wave stores its quadrant of
// the split's partial directly.
constexpr int kWgWideRows = 128;

template <int PRO>
__global__ __launch_bounds__(kPwThreads, 2) void pw_wgrad_wide_kernel(const bf16_t* __restrict__ dy,
                                                                      const bf16_t* __restrict__ x,
                                                                      float* __restrict__ partial, PwWGeom g) {
  constexpr int RM = kWgWideRows, RK = kWgWideRows, ROWS = RM + RK;
  constexpr int NLD = ROWS * (kWgStage / 8) / kPwThreads;  // 16 loads of 16 bytes per thread per stage
  static_assert(NLD * kPwThreads == ROWS * (kWgStage / 8), "rows must fill the workgroup");
  extern __shared__ __align__(16) uint16_t wg_lds[];
  uint16_t* const tile = wg_lds;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 15, q = lane >> 4;
  const int64_t lin = xcd_swizzle(blockIdx.x, gridDim.x);
  const int tl = static_cast<int>(lin % (g.mblocks * g.kblocks));
  const int64_t rest = lin / (g.mblocks * g.kblocks);
  const int split = static_cast<int>(rest % g.splits);
  const int64_t n = rest / g.splits;
  const int m0 = (tl / g.kblocks) * RM;
  const int k0 = (tl % g.kblocks) * RK;
  const uint32_t V = g.V;
  const __amdgpu_buffer_rsrc_t dr = slab_rsrc(dy + n * g.M * static_cast<int64_t>(V), g.M * V * 2u);
  const __amdgpu_buffer_rsrc_t xr = slab_rsrc(x + n * g.K * static_cast<int64_t>(V), g.K * V * 2u);
  const uint32_t vbeg = static_cast<uint32_t>(split) * g.span;
  const uint32_t vend = min(V, vbeg + g.span);
  const bool do_bias = k0 == 0;

  // Load slot u: tile row r = tid / 16 + 16 u (slots 0-7 dY rows, 8-15 X
  // rows), voxels 8 (tid % 16) .. + 7 of the stage.
  const int grp = threadIdx.x & 15;
  uint32_t rbase[NLD];
  bool rok[NLD];
#pragma unroll
  for (int u = 0; u < NLD; ++u) {
    const int r = (threadIdx.x >> 4) + 16 * u;
    const int row = r < RM ? m0 + r : k0 + (r - RM);
    rok[u] = r < RM ? row < g.M : row < g.K;
    rbase[u] = static_cast<uint32_t>(rok[u] ? row : 0) * V * 2u;
  }
  auto load = [&](uint32_t v, uint4 (&regs)[NLD]) {
    const uint32_t vv = v + 8u * grp;
    const uint32_t nv = vv < vend ? min(8u, vend - vv) : 0u;
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const __amdgpu_buffer_rsrc_t rs = u < NLD / 2 ? dr : xr;
      if (nv == 8u || nv == 0u) {
        regs[u] = buf_load16(rs, nv != 0u && rok[u] ? rbase[u] + vv * 2u : kOob);
      } else {
        regs[u] = load_group(rs, rbase[u] + vv * 2u, rok[u] ? nv : 0u);
      }
    }
  };
  float dbs[NLD / 2];
#pragma unroll
  for (int u = 0; u < NLD / 2; ++u) dbs[u] = 0.f;
  auto stash = [&](const uint4 (&regs)[NLD]) {
#pragma unroll
    for (int u = 0; u < NLD; ++u) {
      const int r = (threadIdx.x >> 4) + 16 * u;
      uint4 v = regs[u];
      if (u < NLD / 2) {
        if (do_bias) {
          dbs[u] += (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) +
                    (bf16_lo(v.z) + bf16_hi(v.z)) + (bf16_lo(v.w) + bf16_hi(v.w));
        }
      } else if (PRO == MEDNEXT_PW_PROLOGUE_GELU) {
        v = gelu_vec(v);  // gelu(0) = 0: missing voxels stay zero
      }
      *reinterpret_cast<uint4*>(tile + r * kWgPitch + 8 * grp) = v;
    }
  };

  const int wm = wave >> 1, wk = wave & 1;  // this wave's 64 x 64 quadrant
  f32x4_t acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 regs[NLD];
  uint32_t v = vbeg;
  load(v, regs);
  while (v < vend) {
    stash(regs);
    __syncthreads();
    load(v + kWgStage, regs);  // next stage in flight during the MFMAs
#pragma unroll
    for (int st = 0; st < kWgStage / 32; ++st) {
      uint4 bf[4];
#pragma unroll
      for (int b = 0; b < 4; ++b)
        bf[b] = *reinterpret_cast<const uint4*>(tile + (RM + 64 * wk + 16 * b + c) * kWgPitch + 32 * st + 8 * q);
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        const uint4 af = *reinterpret_cast<const uint4*>(tile + (64 * wm + 16 * a + c) * kWgPitch + 32 * st + 8 * q);
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma16x16x32(af, bf[b], acc[a][b]);
      }
    }
    __syncthreads();
    v += kWgStage;
  }

  float* out = partial + (n * g.splits + split) * g.stride;
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + 64 * wm + 16 * a + 4 * q + r;
      if (m >= g.M) continue;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int k = k0 + 64 * wk + 16 * b + c;
        if (k < g.K) out[static_cast<int64_t>(m) * g.K + k] = acc[a][b][r];
      }
    }
  if (do_bias) {
    // Row sums: the 16 threads of a row are 16 consecutive lanes of one wave.
#pragma unroll
    for (int u = 0; u < NLD / 2; ++u) {
      float sum = dbs[u];
      sum += __shfl_xor(sum, 1);
      sum += __shfl_xor(sum, 2);
      sum += __shfl_xor(sum, 4);
      sum += __shfl_xor(sum, 8);
      const int m = m0 + (threadIdx.x >> 4) + 16 * u;
      if (grp == 0 && m < g.M) out[static_cast<int64_t>(g.M) * g.K + m] = sum;
    }
  }
}

// dW / dB = fixed-order fp64 sum of the per-split fp32 partials, rounded to
// bf16, in one launch. Partials are [slot][M * K + M]. A block covers OUT
// consecutive outputs with W waves; each wave holds 64 / OUT lane groups, so
// the block has G = W * 64 / OUT groups, and lane group g reads OUT
// consecutive floats of slots g, g + G, ... (summed in slot order). The G
// group sums of each output are then added in group order. The host picks
// OUT (64, 32 or 16) so the grid reaches kFinMinBlocks where the outputs allow
// it, and W so each lane sums at most about kFinSlotsPerLane slots.
constexpr int kFinMinBlocks = 512;
constexpr int kFinSlotsPerLane = 16;
constexpr int kFinMaxWaves = 16;

// AFFINE / NORM weight gradient. The product kernels run on the raw X; with
// X' = (x - c) s + t per (sample, channel k), sum_v dY[m][v] X'[k][v] =
// s P[m][k] + (t - c s) B[m], P = sum_v dY[m][v] x[k][v] and B = sum_v dY[m][v]
// (the bias column of the same partial slot), so each slot's pair is mapped
// with its sample's record while it is summed (fp64). Exact where the folded
// forward rounds X' to bf16.
struct WgradAffine {
  const double* coef;  // [N][K][4] records (null: plain product)
  int64_t k;
  int64_t splits;  // partial slots per sample
  int centred;
};

template <int OUT>
__global__ __launch_bounds__(64 * kFinMaxWaves) void pw_wgrad_reduce_kernel(const float* __restrict__ partial,
                                                                          bf16_t* __restrict__ dw,
                                                                          bf16_t* __restrict__ db, int64_t mk,
                                                                          int64_t m, int64_t slots,
                                                                          int64_t stride, WgradAffine af) {
  extern __shared__ double group_sums[];  // [G][OUT]
  constexpr int kSub = 64 / OUT;
  const int lane = threadIdx.x & 63, o = lane % OUT;
  const int g = (threadIdx.x >> 6) * kSub + lane / OUT;
  const int groups = static_cast<int>(blockDim.x >> 6) * kSub;
  const int64_t total = mk + m;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * OUT + o;
  double s = 0.0;
  if (e < total) {
    const float* p = partial + e;
    if (af.coef != nullptr && e < mk) {
      // Slots are sample-major (splits per sample): this thread's slots of
      // one sample are summed first, then mapped with that sample's record.
      const int64_t row = e / af.k, col = e - row * af.k;
      const float* pb = partial + mk + row;
      int64_t t = g;
      for (int64_t smp = 0; t < slots; ++smp) {
        const int64_t end = min(slots, (smp + 1) * af.splits);
        double sp = 0.0, sb = 0.0;
        for (; t < end; t += groups) {
          sp += p[t * stride];
          sb += pb[t * stride];
        }
        const double* r = af.coef + (smp * af.k + col) * 4;
        const double sc = static_cast<double>(static_cast<float>(r[0]));
        const double sh = static_cast<double>(static_cast<float>(r[1])) -
                          (af.centred ? static_cast<double>(static_cast<float>(r[2])) * sc : 0.0);
        s += sc * sp + sh * sb;
      }
    } else {
#pragma unroll 8
      for (int64_t t = g; t < slots; t += groups) s += p[t * stride];
    }
  }
  group_sums[g * OUT + o] = s;
  __syncthreads();
  if (threadIdx.x < OUT && e < total && (e < mk || db != nullptr)) {
    double acc = 0.0;
    for (int gi = 0; gi < groups; ++gi) acc += group_sums[gi * OUT + o];
    const uint16_t v = f32_to_bf16(static_cast<float>(acc));
    if (e < mk) {
      dw[e].bits = v;
    } else {
      db[e - mk].bits = v;
    }
  }
}

bool aligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) == 0; }

int check_pw_shape(int64_t n, int64_t k, int64_t m, int64_t v, int32_t dtype) {
  MEDNEXT_CHECK_ARG(dtype == MEDNEXT_DTYPE_BF16, "pointwise kernels take bfloat16 tensors");
  MEDNEXT_CHECK_ARG(n >= 1 && k >= 1 && m >= 1 && v >= 1, "empty pointwise problem");
  MEDNEXT_CHECK_ARG(k * v * 2 < (int64_t{1} << 31) && m * v * 2 < (int64_t{1} << 31),
                    "one sample's tensor must be < 2 GiB");
  MEDNEXT_CHECK_ARG(n <= (int64_t{1} << 20), "batch too large");
  return MEDNEXT_STATUS_OK;
}

using FwdKernel = void (*)(const bf16_t*, const bf16_t*, const bf16_t*, const bf16_t*, bf16_t*, PwGeom, PwExtra);

constexpr int kSplitKSlices = 8;  // K >= 256: the four waves of a workgroup split K

// Supported (prologue, epilogue) pairs: NONE with any epilogue, GELU with
// BIAS .. GELU_GRAD, AFFINE with BIAS, BIAS_GELU, BIAS_RESIDUAL or
// BIAS_GELU_PAIR (a GroupNorm or GRN folded into the GEMM that consumes it).
bool pro_epi_supported(int pro, int epi) {
  if (pro == MEDNEXT_PW_PROLOGUE_NONE) return epi >= MEDNEXT_PW_EPILOGUE_BIAS && epi <= MEDNEXT_PW_EPILOGUE_AUX_SCALE;
  if (pro == MEDNEXT_PW_PROLOGUE_GELU) return epi >= MEDNEXT_PW_EPILOGUE_BIAS && epi <= MEDNEXT_PW_EPILOGUE_GELU_GRAD;
  if (pro == MEDNEXT_PW_PROLOGUE_AFFINE) {
    return epi == MEDNEXT_PW_EPILOGUE_BIAS || epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU ||
           epi == MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL || epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR;
  }
  return false;
}

template <int MT>
FwdKernel splitk_instance(int pro, int epi) {
  if (pro == MEDNEXT_PW_PROLOGUE_AFFINE) {
    switch (epi) {
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_splitk_kernel<MT, 2, 1>;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_splitk_kernel<MT, 2, 2>;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_splitk_kernel<MT, 2, 6>;
      default: return pw_fwd_splitk_kernel<MT, 2, 0>;
    }
  }
  if (pro == MEDNEXT_PW_PROLOGUE_GELU) {
    switch (epi) {
      case MEDNEXT_PW_EPILOGUE_BIAS: return pw_fwd_splitk_kernel<MT, 1, 0>;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_splitk_kernel<MT, 1, 1>;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_splitk_kernel<MT, 1, 2>;
      default: return pw_fwd_splitk_kernel<MT, 1, 3>;
    }
  }
  switch (epi) {
    case MEDNEXT_PW_EPILOGUE_BIAS: return pw_fwd_splitk_kernel<MT, 0, 0>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_splitk_kernel<MT, 0, 1>;
    case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_splitk_kernel<MT, 0, 2>;
    case MEDNEXT_PW_EPILOGUE_GELU_GRAD: return pw_fwd_splitk_kernel<MT, 0, 3>;
    case MEDNEXT_PW_EPILOGUE_ROW_REDUCE: return pw_fwd_splitk_kernel<MT, 0, 4>;
    case MEDNEXT_PW_EPILOGUE_AFFINE_SCALE: return pw_fwd_splitk_kernel<MT, 0, 5>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_splitk_kernel<MT, 0, 6>;
    default: return pw_fwd_splitk_kernel<MT, 0, 7>;
  }
}

// Four-tile row groups are only used by epilogues without an aux tensor.
template <int KS, int MT>
FwdKernel fwd_instance_noaux(int pro, int epi) {
  if (pro == MEDNEXT_PW_PROLOGUE_AFFINE) {
    return epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR ? pw_fwd_kernel<KS, MT, 2, 6>
           : epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU    ? pw_fwd_kernel<KS, MT, 2, 1>
                                                     : pw_fwd_kernel<KS, MT, 2, 0>;
  }
  if (epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR) return pw_fwd_kernel<KS, MT, 0, 6>;
  if (pro == MEDNEXT_PW_PROLOGUE_GELU) {
    return epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU ? pw_fwd_kernel<KS, MT, 1, 1> : pw_fwd_kernel<KS, MT, 1, 0>;
  }
  return epi == MEDNEXT_PW_EPILOGUE_BIAS_GELU ? pw_fwd_kernel<KS, MT, 0, 1> : pw_fwd_kernel<KS, MT, 0, 0>;
}

template <int KS, int MT>
FwdKernel fwd_instance(int pro, int epi) {
  if (pro == MEDNEXT_PW_PROLOGUE_AFFINE) {
    switch (epi) {
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_kernel<KS, MT, 2, 1>;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_kernel<KS, MT, 2, 2>;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_kernel<KS, MT, 2, 6>;
      default: return pw_fwd_kernel<KS, MT, 2, 0>;
    }
  }
  if (pro == MEDNEXT_PW_PROLOGUE_GELU) {
    switch (epi) {
      case MEDNEXT_PW_EPILOGUE_BIAS: return pw_fwd_kernel<KS, MT, 1, 0>;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_kernel<KS, MT, 1, 1>;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_kernel<KS, MT, 1, 2>;
      default: return pw_fwd_kernel<KS, MT, 1, 3>;
    }
  }
  switch (epi) {
    case MEDNEXT_PW_EPILOGUE_BIAS: return pw_fwd_kernel<KS, MT, 0, 0>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_kernel<KS, MT, 0, 1>;
    case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_kernel<KS, MT, 0, 2>;
    case MEDNEXT_PW_EPILOGUE_GELU_GRAD: return pw_fwd_kernel<KS, MT, 0, 3>;
    case MEDNEXT_PW_EPILOGUE_ROW_REDUCE: return pw_fwd_kernel<KS, MT, 0, 4>;
    case MEDNEXT_PW_EPILOGUE_AFFINE_SCALE: return pw_fwd_kernel<KS, MT, 0, 5>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_kernel<KS, MT, 0, 6>;
    default: return pw_fwd_kernel<KS, MT, 0, 7>;
  }
}

// Row-group height: four m-tiles (the whole 64-row output of the K = 32
// expansions, so X is read once) when the epilogue reads no aux tensor;
// otherwise two (accumulators + aux registers stay within two waves
// per SIMD), one when the weight block would not fit the LDS budget.
int pick_mt(int64_t k, int64_t m, int epi) {
  const int64_t ks = cdiv(k, 32);
  const bool aux = epi_has_aux(epi);
  auto fits = [&](int mt) { return static_cast<size_t>(16 * mt) * ks * 32 * 2 <= kMaxWeightLds; };
  if (ks >= kSplitKSlices) return m > 16 && fits(2) ? 2 : 1;
  // Two aux rows per output row: two m-tiles fit the register budget only with
  // the single-slice loop unrolled (K <= 32).
  if (epi == MEDNEXT_PW_EPILOGUE_AFFINE_SCALE) return ks == 1 && m > 16 && fits(2) ? 2 : 1;
  // MT = 4 is instantiated for a single K slice only (pick_fwd).
  if (!aux && ks == 1 && m > 32 && fits(4)) return 4;
  if (m > 16 && fits(2)) return 2;
  return 1;
}

template <int MT>
FwdKernel tiled_instance(int pro, int epi) {
  if (pro == MEDNEXT_PW_PROLOGUE_AFFINE) {
    switch (epi) {
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_tiled_kernel<MT, 2, 1>;
      case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_tiled_kernel<MT, 2, 2>;
      case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_tiled_kernel<MT, 2, 6>;
      default: return pw_fwd_tiled_kernel<MT, 2, 0>;
    }
  }
  switch (epi) {
    case MEDNEXT_PW_EPILOGUE_BIAS: return pw_fwd_tiled_kernel<MT, 0, 0>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_fwd_tiled_kernel<MT, 0, 1>;
    case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_fwd_tiled_kernel<MT, 0, 2>;
    case MEDNEXT_PW_EPILOGUE_GELU_GRAD: return pw_fwd_tiled_kernel<MT, 0, 3>;
    case MEDNEXT_PW_EPILOGUE_AFFINE_SCALE: return pw_fwd_tiled_kernel<MT, 0, 5>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_fwd_tiled_kernel<MT, 0, 6>;
    default: return pw_fwd_tiled_kernel<MT, 0, 7>;
  }
}

// Shapes and modes the tiled product takes: whole 32-channel slices, whole
// 16-row fragments, no GELU prologue (its K is always small here) and no
// ROW_REDUCE (its slots are per streaming workgroup).
bool tiled_eligible(int64_t k, int64_t m, int pro, int epi) {
  return k % 32 == 0 && m % 16 == 0 && pro != MEDNEXT_PW_PROLOGUE_GELU && epi != MEDNEXT_PW_EPILOGUE_ROW_REDUCE;
}

FwdKernel pick_fwd(int64_t k, int mt, int pro, int epi) {
  const int64_t ks = cdiv(k, 32);
  if (ks >= kSplitKSlices) return mt == 1 ? splitk_instance<1>(pro, epi) : splitk_instance<2>(pro, epi);
  if (mt == 4) return fwd_instance_noaux<1, 4>(pro, epi);
  if (mt == 1) return fwd_instance<0, 1>(pro, epi);
  switch (ks) {
    case 1: return fwd_instance<1, 2>(pro, epi);
    case 2: return fwd_instance<2, 2>(pro, epi);
    case 3: return fwd_instance<3, 2>(pro, epi);
    case 4: return fwd_instance<4, 2>(pro, epi);
    default: return fwd_instance<0, 2>(pro, epi);
  }
}

using WgradKernel = void (*)(const bf16_t*, const bf16_t*, float*, PwWGeom);

template <int TM, int TK>
WgradKernel wgrad_instance(int pro) {
  return pro == MEDNEXT_PW_PROLOGUE_GELU ? pw_wgrad_kernel<TM, TK, 1> : pw_wgrad_kernel<TM, TK, 0>;
}

// 16-row/column tiles per workgroup side: up to four, fewer when the matrix is
// narrower (so no MFMA works on rows that do not exist).
int tiles_for(int64_t rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : 4; }

WgradKernel pick_wgrad(int tm, int tk, int pro) {
  switch (tm * 8 + tk) {
    case 1 * 8 + 1: return wgrad_instance<1, 1>(pro);
    case 1 * 8 + 2: return wgrad_instance<1, 2>(pro);
    case 1 * 8 + 4: return wgrad_instance<1, 4>(pro);
    case 2 * 8 + 1: return wgrad_instance<2, 1>(pro);
    case 2 * 8 + 2: return wgrad_instance<2, 2>(pro);
    case 2 * 8 + 4: return wgrad_instance<2, 4>(pro);
    case 4 * 8 + 1: return wgrad_instance<4, 1>(pro);
    case 4 * 8 + 2: return wgrad_instance<4, 2>(pro);
    default: return wgrad_instance<4, 4>(pro);
  }
}

}  // namespace
}  // namespace mednext

using namespace mednext;

namespace {

// Launch shape of one forward / transposed product (shared by the launch and
// the ROW_REDUCE slot query).
struct FwdPlan {
  PwGeom g;
  int mt;
  bool splitk;
  int64_t blocks;
  int slots;  // ROW_REDUCE slots per (sample, row)
};

FwdPlan plan_fwd(int64_t n, int64_t k, int64_t m, int64_t v, int epi, int32_t blocks_per_sample) {
  FwdPlan p;
  p.mt = pick_mt(k, m, epi);
  PwGeom& g = p.g;
  g.K = static_cast<int>(k);
  g.M = static_cast<int>(m);
  g.ks = static_cast<int>(cdiv(k, 32));
  g.V = static_cast<uint32_t>(v);
  g.chunks = static_cast<int>(cdiv(v, kChunk));
  g.mgroups = static_cast<int>(cdiv(m, 16 * p.mt));
  g.wt = 0;
  g.ksplit = 1;
  g.kslices = g.ks;
  p.splitk = g.ks >= kSplitKSlices;
  const int64_t groups = n * g.mgroups;
  // Every wave (split-K: every workgroup) gets at least one chunk. The grid
  // stays within the resident workgroups (rounded down): workgroups carry
  // equal shares, so one past them runs as a second round of its own
  // (64^3 64 -> 192: 513 workgroups 62.0 us, 510 49.8 us).
  const int64_t most = p.splitk ? g.chunks : cdiv(g.chunks, 4);
  const int64_t wanted = blocks_per_sample > 0 ? blocks_per_sample : std::max<int64_t>(1, kResidentWgs / groups);
  g.wgs = static_cast<int>(std::max<int64_t>(1, std::min(wanted, most)));
  p.blocks = groups * g.wgs;
  p.slots = p.splitk ? g.wgs : 4 * g.wgs;
  return p;
}

// Process-wide choice between the streaming and the tiled forward kernels
// (MEDNEXT_PW_KERNELS_*), for measurement and tests.
std::atomic<int> g_product_kernels{MEDNEXT_PW_KERNELS_AUTO};

// Automatic choice: the tiled product for the deep products the streaming
// plan would split over K (K >= 256) when that plan reads X at least twice
// (one pass per 16 MT-row group) and the tiled grid still fills the chip.
// Measured on MI355X at the MedNeXt shapes: the tiled kernel takes 0.35-0.7
// of the split-K time there, but loses at K <= 128 with aux-reading
// epilogues (their time is the epilogue's traffic, which the persistent
// streaming kernels overlap better) and on grids of under 256 workgroups.
constexpr int kTiledMinRereads = 2;
constexpr int64_t kTiledMinBlocks = 256;

int64_t tiled_blocks(int64_t n, int64_t m, int64_t v, int mt) { return n * cdiv(m, 64 * mt) * cdiv(v, kChunk); }

// 128-row workgroups (X read once per 128 rows) unless M <= 64 or they would
// leave the chip short of workgroups; then 64-row ones.
int tiled_mt(int64_t n, int64_t m, int64_t v) {
  return m > 64 && tiled_blocks(n, m, v, 2) >= kTiledMinBlocks ? 2 : 1;
}

bool tiled_pays(const FwdPlan& p, int64_t n, int64_t m, int64_t v) {
  return p.splitk && p.g.mgroups >= kTiledMinRereads && tiled_blocks(n, m, v, tiled_mt(n, m, v)) >= kTiledMinBlocks;
}

// The tiled product's launch: row-group height and, for grids short of
// kTiledMinBlocks workgroups, the K ranges that bring them to twice that
// (each range at least one two-slice step).
struct TiledPlan {
  bool tiled;
  int mt;
  int ksplit, kslices;
  size_t kpart_bytes;  // fp32 partials of the K-split (0 without one)
};

// K above kMaxK (the streaming kernels' LDS weight block) only runs tiled,
// without the AFFINE prologue (its per-channel coefficients sit in LDS).
bool tiled_only(int64_t k) { return k > kMaxK; }

TiledPlan plan_tiled(int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue, int32_t epilogue, bool allow_split) {
  TiledPlan t{false, 1, 1, static_cast<int>(k / 32), 0};
  if (prologue == MEDNEXT_PW_PROLOGUE_NORM) prologue = MEDNEXT_PW_PROLOGUE_AFFINE;  // same kernels
  if (n < 1 || k < 1 || k > kMaxTiledK || m < 1 || v < 1 || !pro_epi_supported(prologue, epilogue)) return t;
  if (tiled_only(k) && prologue == MEDNEXT_PW_PROLOGUE_AFFINE) return t;
  const int choice = g_product_kernels.load(std::memory_order_relaxed);
  if (choice == MEDNEXT_PW_KERNELS_STREAMING || !tiled_eligible(k, m, prologue, epilogue)) return t;
  t.mt = choice == MEDNEXT_PW_KERNELS_TILED_64 ? 1 : tiled_mt(n, m, v);
  const FwdPlan p = plan_fwd(n, k, m, v, epilogue, 0);
  const int64_t blocks = tiled_blocks(n, m, v, t.mt);
  const int ks = static_cast<int>(k / 32);
  int split = 1;
  if (allow_split && blocks < kTiledMinBlocks && ks >= 2 * kTileSlices) {
    split = static_cast<int>(std::min<int64_t>(cdiv(2 * kTiledMinBlocks, blocks), ks / kTileSlices));
  }
  t.kslices = static_cast<int>(cdiv(ks, split));
  t.ksplit = static_cast<int>(cdiv(ks, t.kslices));
  if (choice == MEDNEXT_PW_KERNELS_TILED || choice == MEDNEXT_PW_KERNELS_TILED_64 || tiled_only(k)) {
    t.tiled = true;
  } else {
    t.tiled = tiled_pays(p, n, m, v) || (p.splitk && t.ksplit > 1);
  }
  if (!t.tiled || t.ksplit == 1) {
    t.ksplit = 1;
    t.kslices = ks;
  } else {
    t.kpart_bytes = static_cast<size_t>(n) * t.ksplit * m * (cdiv(v, 8) * 8) * sizeof(float);
  }
  return t;
}

using KsplitEpilogue = void (*)(const bf16_t*, const bf16_t*, bf16_t*, PwGeom, PwExtra, int64_t);

KsplitEpilogue ksplit_epilogue(int epi) {
  switch (epi) {
    case MEDNEXT_PW_EPILOGUE_BIAS: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_BIAS>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_BIAS_GELU>;
    case MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL>;
    case MEDNEXT_PW_EPILOGUE_GELU_GRAD: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_GELU_GRAD>;
    case MEDNEXT_PW_EPILOGUE_AFFINE_SCALE: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_AFFINE_SCALE>;
    case MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR>;
    default: return pw_ksplit_epilogue_kernel<MEDNEXT_PW_EPILOGUE_AUX_SCALE>;
  }
}

int32_t launch_tiled(const void* x, const void* weight, const void* bias, const void* aux, void* y, PwExtra ex,
                     int64_t n, int64_t k, int64_t m, int64_t v, int32_t weight_layout, int32_t prologue,
                     int32_t epilogue, const TiledPlan& t, void* workspace, void* stream) {
  const int mt = t.mt;
  PwGeom g{};
  g.K = static_cast<int>(k);
  g.M = static_cast<int>(m);
  g.ks = static_cast<int>(k / 32);
  g.V = static_cast<uint32_t>(v);
  g.chunks = static_cast<int>(cdiv(v, kChunk));
  g.mgroups = static_cast<int>(cdiv(m, 64 * mt));
  g.wgs = 1;
  g.wt = weight_layout;
  g.ksplit = t.ksplit;
  g.kslices = t.kslices;
  ex.kpart = static_cast<float*>(workspace);
  const int64_t blocks = n * g.mgroups * g.chunks * g.ksplit;
  MEDNEXT_CHECK_ARG(blocks < (int64_t{1} << 31), "grid too large");
  const int64_t sps = std::min<int64_t>(kTileSlices, g.kslices);
  const int64_t nstages = g.kslices > kTileSlices ? 2 : 1;
  const size_t slice = static_cast<size_t>(8 * 64 + 4 * mt * 64) * 16;
  const size_t lds = static_cast<size_t>(nstages * sps) * slice + 3 * 64 * mt * sizeof(float) +
                     (prologue == MEDNEXT_PW_PROLOGUE_AFFINE ? 3 * static_cast<size_t>(k) * sizeof(float) : 0);
  FwdKernel fn = mt == 1 ? tiled_instance<1>(prologue, epilogue) : tiled_instance<2>(prologue, epilogue);
  const auto st = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(kPwThreads), lds, st,
                     static_cast<const bf16_t*>(x), static_cast<const bf16_t*>(weight),
                     static_cast<const bf16_t*>(bias), static_cast<const bf16_t*>(aux), static_cast<bf16_t*>(y), g, ex);
  MEDNEXT_CHECK_LAUNCH();
  if (g.ksplit > 1) {
    const int64_t threads = n * m * cdiv(v, 8);
    hipLaunchKernelGGL(ksplit_epilogue(epilogue), dim3(static_cast<unsigned>(cdiv(threads, kPwThreads))),
                       dim3(kPwThreads), 0, st, static_cast<const bf16_t*>(bias), static_cast<const bf16_t*>(aux),
                       static_cast<bf16_t*>(y), g, ex, n);
    MEDNEXT_CHECK_LAUNCH();
  }
  return MEDNEXT_STATUS_OK;
}

}  // namespace

extern "C" int32_t mednext_pointwise_set_kernels(int32_t choice) {
  MEDNEXT_CHECK_ARG(choice >= MEDNEXT_PW_KERNELS_AUTO && choice <= MEDNEXT_PW_KERNELS_TILED_64,
                    "choice must be MEDNEXT_PW_KERNELS_AUTO, _STREAMING, _TILED or _TILED_64");
  g_product_kernels.store(choice, std::memory_order_relaxed);
  return MEDNEXT_STATUS_OK;
}

extern "C" int32_t mednext_pointwise_uses_tiled(int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                                int32_t epilogue) {
  return plan_tiled(n, k, m, v, prologue, epilogue, false).tiled ? 1 : 0;
}

extern "C" size_t mednext_pointwise_fwd_workspace_bytes(int64_t n, int64_t k, int64_t m, int64_t v,
                                                        int32_t prologue, int32_t epilogue) {
  return plan_tiled(n, k, m, v, prologue, epilogue, true).kpart_bytes;
}

extern "C" int64_t mednext_pointwise_row_slots(int64_t n, int64_t k, int64_t m, int64_t v,
                                               int32_t blocks_per_sample) {
  if (n < 1 || k < 1 || k > kMaxK || m < 1 || v < 1 || blocks_per_sample < 0) return 0;
  return plan_fwd(n, k, m, v, MEDNEXT_PW_EPILOGUE_ROW_REDUCE, blocks_per_sample).slots;
}

extern "C" int32_t mednext_pointwise_fwd_ws(const void* x, const void* weight, const void* bias, const void* aux,
                                            const void* aux2, void* y, void* y2, int64_t n, int64_t k, int64_t m,
                                            int64_t v, int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                            const void* prologue_coef, const void* epilogue_coef,
                                            void* row_partial, int32_t dtype, int32_t blocks_per_sample,
                                            void* workspace, size_t workspace_bytes, void* stream) {
  if (int st = check_pw_shape(n, k, m, v, dtype)) return st;
  // NORM runs the AFFINE kernels with the records' centre subtracted first.
  const int centred = prologue == MEDNEXT_PW_PROLOGUE_NORM ? 1 : 0;
  if (centred) prologue = MEDNEXT_PW_PROLOGUE_AFFINE;
  const bool reduce = epilogue == MEDNEXT_PW_EPILOGUE_ROW_REDUCE;
  MEDNEXT_CHECK_ARG(x != nullptr && weight != nullptr && (y != nullptr || reduce), "null tensor pointer");
  MEDNEXT_CHECK_ARG(weight_layout == 0 || weight_layout == 1, "weight_layout must be 0 ([M][K]) or 1 ([K][M])");
  MEDNEXT_CHECK_ARG(pro_epi_supported(prologue, epilogue), "unsupported prologue / epilogue combination");
  MEDNEXT_CHECK_ARG(!epi_has_aux(epilogue) || aux != nullptr, "this epilogue needs the aux tensor");
  MEDNEXT_CHECK_ARG(epilogue != MEDNEXT_PW_EPILOGUE_AFFINE_SCALE || aux2 != nullptr, "AFFINE_SCALE needs aux2");
  MEDNEXT_CHECK_ARG(epilogue != MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR || y2 != nullptr, "BIAS_GELU_PAIR needs y2");
  MEDNEXT_CHECK_ARG(prologue != MEDNEXT_PW_PROLOGUE_AFFINE || (prologue_coef != nullptr && aligned(prologue_coef, 8)),
                    "the AFFINE / NORM prologue needs 8-byte aligned coefficient records");
  MEDNEXT_CHECK_ARG(prologue != MEDNEXT_PW_PROLOGUE_AFFINE || weight_layout == 0,
                    "the AFFINE / NORM prologue takes a [M][K] weight");
  MEDNEXT_CHECK_ARG(epilogue != MEDNEXT_PW_EPILOGUE_AFFINE_SCALE ||
                        (epilogue_coef != nullptr && aligned(epilogue_coef, 8)),
                    "the AFFINE_SCALE epilogue needs 8-byte aligned coefficients");
  MEDNEXT_CHECK_ARG(!reduce || (row_partial != nullptr && aligned(row_partial, 8)),
                    "the ROW_REDUCE epilogue needs an 8-byte aligned row_partial buffer");
  MEDNEXT_CHECK_ARG(aligned(x, 2) && (y == nullptr || aligned(y, 2)) && (aux == nullptr || aligned(aux, 2)) &&
                        (aux2 == nullptr || aligned(aux2, 2)) && (y2 == nullptr || aligned(y2, 2)) &&
                        aligned(weight, 16) && (bias == nullptr || aligned(bias, 2)),
                    "pointwise tensors must be bf16-aligned and the weight 16-byte aligned");
  MEDNEXT_CHECK_ARG(blocks_per_sample >= 0, "blocks_per_sample must be >= 0 (0 = automatic)");
  PwExtra ex{static_cast<const double*>(prologue_coef), centred, static_cast<const double*>(epilogue_coef),
             static_cast<double*>(row_partial), static_cast<const bf16_t*>(aux2), static_cast<bf16_t*>(y2), 0,
             nullptr};
  if (blocks_per_sample == 0) {
    // The K-split tiled product when the caller's workspace holds its partials.
    TiledPlan t = plan_tiled(n, k, m, v, prologue, epilogue, true);
    if (t.ksplit > 1 && (workspace == nullptr || workspace_bytes < t.kpart_bytes || !aligned(workspace, 16)))
      t = plan_tiled(n, k, m, v, prologue, epilogue, false);
    if (t.tiled)
      return launch_tiled(x, weight, bias, aux, y, ex, n, k, m, v, weight_layout, prologue, epilogue, t, workspace,
                          stream);
  }
  MEDNEXT_CHECK_ARG(k <= kMaxK,
                    "input channels above 2048 take the tiled product only (K <= 8192 and a multiple of 32, M a "
                    "multiple of 16, no GELU / AFFINE / NORM prologue or ROW_REDUCE epilogue, AUTO or TILED "
                    "kernels, blocks_per_sample 0)");
  FwdPlan p = plan_fwd(n, k, m, v, epilogue, blocks_per_sample);
  p.g.wt = weight_layout;
  ex.slots = p.slots;
  MEDNEXT_CHECK_ARG(p.blocks < (int64_t{1} << 31), "grid too large");
  MEDNEXT_CHECK_ARG(p.mt != 4 || p.g.ks == 1, "internal: 64-row groups take one 32-channel K slice");
  const int mt = p.mt;
  const size_t lds = static_cast<size_t>(16 * mt) * p.g.ks * 32 * 2 + kRowVecs * 16 * mt * sizeof(float) +
                     (p.splitk ? static_cast<size_t>(mt) * 8 * 4 * 64 * sizeof(float) : 0) +
                     (prologue == MEDNEXT_PW_PROLOGUE_AFFINE ? static_cast<size_t>(p.g.ks) * 32 * 3 * sizeof(float) : 0);
  hipLaunchKernelGGL(pick_fwd(k, mt, prologue, epilogue), dim3(static_cast<unsigned>(p.blocks)), dim3(kPwThreads),
                     lds, static_cast<hipStream_t>(stream), static_cast<const bf16_t*>(x),
                     static_cast<const bf16_t*>(weight), static_cast<const bf16_t*>(bias),
                     static_cast<const bf16_t*>(aux), static_cast<bf16_t*>(y), p.g, ex);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

extern "C" int32_t mednext_pointwise_fwd_ex(const void* x, const void* weight, const void* bias, const void* aux,
                                            const void* aux2, void* y, void* y2, int64_t n, int64_t k, int64_t m,
                                            int64_t v, int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                            const void* prologue_coef, const void* epilogue_coef,
                                            void* row_partial, int32_t dtype, int32_t blocks_per_sample,
                                            void* stream) {
  return mednext_pointwise_fwd_ws(x, weight, bias, aux, aux2, y, y2, n, k, m, v, weight_layout, prologue, epilogue,
                                  prologue_coef, epilogue_coef, row_partial, dtype, blocks_per_sample, nullptr, 0,
                                  stream);
}

extern "C" int32_t mednext_pointwise_fwd(const void* x, const void* weight, const void* bias, const void* aux,
                                         void* y, int64_t n, int64_t k, int64_t m, int64_t v,
                                         int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                         int32_t dtype, int32_t blocks_per_sample, void* stream) {
  MEDNEXT_CHECK_ARG(prologue == MEDNEXT_PW_PROLOGUE_NONE || prologue == MEDNEXT_PW_PROLOGUE_GELU, "bad prologue");
  MEDNEXT_CHECK_ARG(epilogue >= MEDNEXT_PW_EPILOGUE_BIAS && epilogue <= MEDNEXT_PW_EPILOGUE_GELU_GRAD, "bad epilogue");
  return mednext_pointwise_fwd_ex(x, weight, bias, aux, nullptr, y, nullptr, n, k, m, v, weight_layout, prologue,
                                  epilogue, nullptr, nullptr, nullptr, dtype, blocks_per_sample, stream);
}

namespace {

// Voxels per split for `splits` splits: whole 128-voxel LDS stages.
int64_t wgrad_span(int64_t v, int32_t splits) { return cdiv(cdiv(v, kWgStage), splits) * kWgStage; }

}  // namespace

namespace {

// Bytes of per-split fp32 partials (a whole number of 8-byte words).
size_t wgrad_partial_bytes(int64_t n, int64_t k, int64_t m, int64_t v, int32_t splits) {
  const int64_t used = cdiv(v, wgrad_span(v, splits));
  return static_cast<size_t>(cdiv(static_cast<int64_t>(n) * used * (m * k + m), 2) * 2) * sizeof(float);
}

}  // namespace

extern "C" size_t mednext_pointwise_wgrad_workspace_bytes(int64_t n, int64_t k, int64_t m, int64_t v,
                                                          int32_t splits) {
  if (n < 1 || k < 1 || m < 1 || v < 1 || splits < 1) return 0;
  return wgrad_partial_bytes(n, k, m, v, splits);
}

extern "C" int32_t mednext_pointwise_wgrad_ex(const void* grad_output, const void* x, void* grad_weight,
                                              void* grad_bias, void* workspace, size_t workspace_bytes,
                                              int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                              const void* prologue_coef, int32_t dtype, int32_t splits,
                                              void* stream) {
  if (int st = check_pw_shape(n, k, m, v, dtype)) return st;
  MEDNEXT_CHECK_ARG(grad_output != nullptr && x != nullptr && grad_weight != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG(prologue == MEDNEXT_PW_PROLOGUE_NONE || prologue == MEDNEXT_PW_PROLOGUE_GELU ||
                        prologue == MEDNEXT_PW_PROLOGUE_AFFINE || prologue == MEDNEXT_PW_PROLOGUE_NORM,
                    "bad prologue");
  const bool affine = prologue == MEDNEXT_PW_PROLOGUE_AFFINE || prologue == MEDNEXT_PW_PROLOGUE_NORM;
  MEDNEXT_CHECK_ARG(!affine || (prologue_coef != nullptr && aligned(prologue_coef, 8)),
                    "the AFFINE / NORM prologue needs 8-byte aligned coefficient records");
  // AFFINE / NORM: the product runs on the raw X and the reduction maps it.
  const WgradAffine af{affine ? static_cast<const double*>(prologue_coef) : nullptr, k, 0,
                       prologue == MEDNEXT_PW_PROLOGUE_NORM ? 1 : 0};
  if (affine) prologue = MEDNEXT_PW_PROLOGUE_NONE;
  MEDNEXT_CHECK_ARG(splits >= 1 && splits <= 65535, "splits must be in [1, 65535]");
  MEDNEXT_CHECK_ARG(aligned(grad_output, 2) && aligned(x, 2) && aligned(grad_weight, 2) &&
                        (grad_bias == nullptr || aligned(grad_bias, 2)),
                    "pointwise tensors must be bf16-aligned");
  const size_t need = mednext_pointwise_wgrad_workspace_bytes(n, k, m, v, splits);
  MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= need, "workspace too small");
  MEDNEXT_CHECK_ARG(aligned(workspace, 8), "workspace must be 8-byte aligned");
  PwWGeom g;
  g.K = static_cast<int>(k);
  g.M = static_cast<int>(m);
  g.V = static_cast<uint32_t>(v);
  g.span = static_cast<uint32_t>(wgrad_span(v, splits));
  g.splits = static_cast<int>(cdiv(v, static_cast<int64_t>(g.span)));
  const int tm = tiles_for(m), tk = tiles_for(k);
  // 128 x 128 tiles where both sides fill them and the grid still has
  // kTiledMinBlocks workgroups (any 64 x 64 shape under TILED).
  const int choice = g_product_kernels.load(std::memory_order_relaxed);
  const int64_t wide_blocks = n * g.splits * cdiv(m, kWgWideRows) * cdiv(k, kWgWideRows);
  const bool wide = choice == MEDNEXT_PW_KERNELS_TILED
                        ? tm == 4 && tk == 4
                        : choice == MEDNEXT_PW_KERNELS_AUTO && m >= kWgWideRows && k >= kWgWideRows &&
                              wide_blocks >= kTiledMinBlocks;
  const int side_m = wide ? kWgWideRows : 16 * tm, side_k = wide ? kWgWideRows : 16 * tk;
  g.mblocks = static_cast<int>(cdiv(m, side_m));
  g.kblocks = static_cast<int>(cdiv(k, side_k));
  g.stride = m * k + m;
  const int64_t blocks = n * g.splits * g.mblocks * static_cast<int64_t>(g.kblocks);
  MEDNEXT_CHECK_ARG(blocks < (int64_t{1} << 31), "grid too large");
  const auto s = static_cast<hipStream_t>(stream);
  auto* part = static_cast<float*>(workspace);
  if (wide) {
    const size_t lds = static_cast<size_t>(2 * kWgWideRows) * kWgPitch * 2;
    WgradKernel fn = prologue == MEDNEXT_PW_PROLOGUE_GELU ? pw_wgrad_wide_kernel<1> : pw_wgrad_wide_kernel<0>;
    hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(blocks)), dim3(kPwThreads), lds, s,
                       static_cast<const bf16_t*>(grad_output), static_cast<const bf16_t*>(x), part, g);
  } else {
    hipLaunchKernelGGL(pick_wgrad(tm, tk, prologue), dim3(static_cast<unsigned>(blocks)), dim3(kPwThreads), 0, s,
                       static_cast<const bf16_t*>(grad_output), static_cast<const bf16_t*>(x), part, g);
  }
  MEDNEXT_CHECK_LAUNCH();
  const int64_t total = m * k + m;
  const int64_t slots = n * g.splits;
  int out = 64;
  while (out > 16 && cdiv(total, static_cast<int64_t>(out)) < kFinMinBlocks) out /= 2;
  const int waves = static_cast<int>(
      std::clamp<int64_t>(cdiv(cdiv(slots, static_cast<int64_t>(kFinSlotsPerLane)), static_cast<int64_t>(64 / out)),
                          1, kFinMaxWaves));
  const dim3 fin_grid(static_cast<unsigned>(cdiv(total, static_cast<int64_t>(out))));
  const size_t fin_lds = static_cast<size_t>(waves) * 64 * sizeof(double);
  auto reduce = out == 64 ? pw_wgrad_reduce_kernel<64> : out == 32 ? pw_wgrad_reduce_kernel<32>
                                                                   : pw_wgrad_reduce_kernel<16>;
  WgradAffine fin_af = af;
  fin_af.splits = g.splits;
  hipLaunchKernelGGL(reduce, fin_grid, dim3(64 * waves), fin_lds, s, part, static_cast<bf16_t*>(grad_weight),
                     static_cast<bf16_t*>(grad_bias), m * k, m, slots, g.stride, fin_af);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

extern "C" int32_t mednext_pointwise_wgrad(const void* grad_output, const void* x, void* grad_weight,
                                           void* grad_bias, void* workspace, size_t workspace_bytes,
                                           int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                           int32_t dtype, int32_t splits, void* stream) {
  MEDNEXT_CHECK_ARG(prologue == MEDNEXT_PW_PROLOGUE_NONE || prologue == MEDNEXT_PW_PROLOGUE_GELU, "bad prologue");
  return mednext_pointwise_wgrad_ex(grad_output, x, grad_weight, grad_bias, workspace, workspace_bytes, n, k, m, v,
                                    prologue, nullptr, dtype, splits, stream);
}
