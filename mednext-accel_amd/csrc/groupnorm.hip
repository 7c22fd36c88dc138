// GroupNorm with groups == channels (per-(n, c) normalisation over the spatial
// volume V), forward and backward, for gfx950.
//
// Each (n, c) row of V elements is split into `splits` contiguous chunks, one
// workgroup per chunk. Statistics use sums shifted by the row's first element
// (robust against a large mean), accumulated in fp32 per thread (fp64 for fp64
// data) and combined in fp64 across waves and across chunks in a fixed order:
// results are bit-reproducible run to run. The apply passes recombine the
// row's partials themselves, so forward is two launches and backward three.
#include "common.h"

namespace mednext {
namespace {

constexpr int kThreads = 256;

// Runtime-typed scalar load for the small per-channel parameter vectors.
__device__ inline double load_param(const void* p, int dtype, int64_t i) {
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: return static_cast<const float*>(p)[i];
    case MEDNEXT_DTYPE_F64: return static_cast<const double*>(p)[i];
    case MEDNEXT_DTYPE_F16: return static_cast<float>(static_cast<const f16_t*>(p)[i]);
    default: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
  }
}
__device__ inline void store_param(void* p, int dtype, int64_t i, double v) {
  switch (dtype) {
    case MEDNEXT_DTYPE_F32: static_cast<float*>(p)[i] = static_cast<float>(v); break;
    case MEDNEXT_DTYPE_F64: static_cast<double*>(p)[i] = v; break;
    case MEDNEXT_DTYPE_F16: static_cast<f16_t*>(p)[i] = static_cast<f16_t>(static_cast<float>(v)); break;
    default: static_cast<uint16_t*>(p)[i] = f32_to_bf16(static_cast<float>(v)); break;
  }
}

struct Chunk {
  int64_t row;    // n * C + c
  int split;
  int64_t begin;  // element range [begin, end) inside the row
  int64_t end;
};

__device__ inline Chunk chunk_of_block(int64_t v, int splits, int64_t chunk) {
  Chunk ck;
  ck.row = blockIdx.x / splits;
  ck.split = static_cast<int>(blockIdx.x % splits);
  ck.begin = static_cast<int64_t>(ck.split) * chunk;
  ck.end = ck.begin + chunk < v ? ck.begin + chunk : v;
  return ck;
}

// Block-wide sum of two doubles in fixed order; result valid in thread 0.
__device__ inline void block_sum2(double& a, double& b) {
  __shared__ double red[kThreads / 64][2];
  a = wave_sum(a);
  b = wave_sum(b);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    red[wave][0] = a;
    red[wave][1] = b;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    a = red[0][0];
    b = red[0][1];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) {
      a += red[w][0];
      b += red[w][1];
    }
  }
}

// Combine a row's `splits` partial pairs (fixed order) into the block's shared
// copy; every thread returns the combined pair.
__device__ inline void combine_row(const double* __restrict__ part, int64_t row, int splits,
                                   double& a, double& b) {
  __shared__ double comb[2];
  if (threadIdx.x == 0) {
    double sa = 0.0, sb = 0.0;
    const double* p = part + row * splits * 2;
    for (int s = 0; s < splits; ++s) {
      sa += p[2 * s];
      sb += p[2 * s + 1];
    }
    comb[0] = sa;
    comb[1] = sb;
  }
  __syncthreads();
  a = comb[0];
  b = comb[1];
}

// Vector loops keep kUnroll 8-element vectors per thread in flight.
constexpr int kUnroll = 4;

template <typename Tx>
__global__ __launch_bounds__(kThreads) void gn_stats_kernel(const Tx* __restrict__ x, int64_t v,
                                                            int splits, int64_t chunk, bool vec_ok,
                                                            double* __restrict__ part) {
  using Acc = typename AccOf<Tx>::type;
  const Chunk ck = chunk_of_block(v, splits, chunk);
  const Tx* __restrict__ row = x + ck.row * v;
  const Acc shift = Cvt<Tx, Acc>::load(row[0]);
  Acc s1 = Acc(0), s2 = Acc(0);
  const Tx* __restrict__ cp = row + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const Acc d = Cvt<Tx, Acc>::load(cp[rs.scalar_index(i)]) - shift;
    s1 += d;
    s2 += d * d;
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc e[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<Tx, Acc>(cp + rs.head + 8 * j, e[u]);
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) e[u][t] = shift;
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const Acc d = e[u][t] - shift;
        s1 += d;
        s2 += d * d;
      }
  }
  double a = s1, b = s2;
  block_sum2(a, b);
  if (threadIdx.x == 0) {
    part[(ck.row * splits + ck.split) * 2] = a;
    part[(ck.row * splits + ck.split) * 2 + 1] = b;
  }
}

template <typename Tx, typename Ty>
__global__ __launch_bounds__(kThreads) void gn_apply_kernel(
    const Tx* __restrict__ x, const void* __restrict__ gamma, const void* __restrict__ beta,
    int pdtype, Ty* __restrict__ y, void* __restrict__ mean_out, void* __restrict__ rstd_out,
    int64_t c, int64_t v, double eps, int splits, int64_t chunk, bool vec_ok, const double* __restrict__ part) {
  using Acc = typename AccOf<Tx>::type;
  const Chunk ck = chunk_of_block(v, splits, chunk);
  const Tx* __restrict__ row = x + ck.row * v;
  Ty* __restrict__ out = y + ck.row * v;
  double s1, s2;
  combine_row(part, ck.row, splits, s1, s2);
  const double shift = static_cast<double>(Cvt<Tx, Acc>::load(row[0]));
  const double inv_n = 1.0 / static_cast<double>(v);
  const double dmean = s1 * inv_n;
  double var = s2 * inv_n - dmean * dmean;
  if (var < 0.0) var = 0.0;
  const double mean = shift + dmean;
  const double rstd = 1.0 / sqrt(var + eps);
  const int64_t ch = ck.row % c;
  const double g = gamma ? load_param(gamma, pdtype, ch) : 1.0;
  const double bt = beta ? load_param(beta, pdtype, ch) : 0.0;
  // y = (x - mean) * (rstd * gamma) + beta
  const Acc scale = static_cast<Acc>(rstd * g);
  const Acc m_acc = static_cast<Acc>(mean);
  const Acc offset = static_cast<Acc>(bt);
  if (ck.split == 0 && threadIdx.x == 0) {
    if (sizeof(Acc) == 8) {
      static_cast<double*>(mean_out)[ck.row] = mean;
      static_cast<double*>(rstd_out)[ck.row] = rstd;
    } else {
      static_cast<float*>(mean_out)[ck.row] = static_cast<float>(mean);
      static_cast<float*>(rstd_out)[ck.row] = static_cast<float>(rstd);
    }
  }
  const Tx* __restrict__ cp = row + ck.begin;
  Ty* __restrict__ op = out + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    op[k] = Cvt<Ty, Acc>::store(fma_acc(Cvt<Tx, Acc>::load(cp[k]) - m_acc, scale, offset));
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc e[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) load8<Tx, Acc>(cp + rs.head + 8 * j, e[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
#pragma unroll
        for (int t = 0; t < 8; ++t) e[u][t] = fma_acc(e[u][t] - m_acc, scale, offset);
        store8<Ty, Acc>(op + rs.head + 8 * j, e[u]);
      }
    }
  }
}

// Statistics only (the normalisation folded into the GEMM that consumes it):
// one thread per (n, c) row combines the row's partials in the fixed order of
// combine_row, computes mean and rstd exactly as gn_apply_kernel does, and
// writes them with the row's record coef[row] = (rstd * gamma, beta, mean,
// rstd) (fp64): taken as floats, fma(x - mean, rstd * gamma, beta) is
// gn_apply_kernel's fp32 expression, so a consumer reproduces its output.
template <typename Tx>
__global__ __launch_bounds__(256) void gn_coef_kernel(const Tx* __restrict__ x, const void* __restrict__ gamma,
                                                      const void* __restrict__ beta, int pdtype,
                                                      void* __restrict__ mean_out, void* __restrict__ rstd_out,
                                                      double* __restrict__ coef, int64_t rows, int64_t c, int64_t v,
                                                      double eps, int splits, const double* __restrict__ part) {
  using Acc = typename AccOf<Tx>::type;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  double s1 = 0.0, s2 = 0.0;
  const double* p = part + row * splits * 2;
  for (int sp = 0; sp < splits; ++sp) {
    s1 += p[2 * sp];
    s2 += p[2 * sp + 1];
  }
  const double shift = static_cast<double>(Cvt<Tx, Acc>::load(x[row * v]));
  const double inv_n = 1.0 / static_cast<double>(v);
  const double dmean = s1 * inv_n;
  double var = s2 * inv_n - dmean * dmean;
  if (var < 0.0) var = 0.0;
  const double mean = shift + dmean;
  const double rstd = 1.0 / sqrt(var + eps);
  const int64_t ch = row % c;
  const double g = gamma ? load_param(gamma, pdtype, ch) : 1.0;
  const double bt = beta ? load_param(beta, pdtype, ch) : 0.0;
  if (sizeof(Acc) == 8) {
    static_cast<double*>(mean_out)[row] = mean;
    static_cast<double*>(rstd_out)[row] = rstd;
  } else {
    static_cast<float*>(mean_out)[row] = static_cast<float>(mean);
    static_cast<float*>(rstd_out)[row] = static_cast<float>(rstd);
  }
  coef[row * 4] = rstd * g;
  coef[row * 4 + 1] = bt;
  coef[row * 4 + 2] = mean;
  coef[row * 4 + 3] = rstd;
}

template <typename Ts>
__device__ inline double load_stat(const void* p, int64_t i) {
  return static_cast<double>(static_cast<const Ts*>(p)[i]);
}

template <typename Tdy, typename Tx>
__global__ __launch_bounds__(kThreads) void gn_bwd_reduce_kernel(
    const Tdy* __restrict__ dy, const Tx* __restrict__ x, const void* __restrict__ mean,
    const void* __restrict__ rstd, int64_t v, int splits, int64_t chunk, bool vec_ok,
    double* __restrict__ part) {
  using Acc = typename AccOf<Tx>::type;
  const Chunk ck = chunk_of_block(v, splits, chunk);
  const Tx* __restrict__ xr = x + ck.row * v;
  const Tdy* __restrict__ gr = dy + ck.row * v;
  const Acc m = static_cast<Acc>(load_stat<Acc>(mean, ck.row));
  const Acc r = static_cast<Acc>(load_stat<Acc>(rstd, ck.row));
  Acc sa = Acc(0), sb = Acc(0);
  const Tx* __restrict__ xp = xr + ck.begin;
  const Tdy* __restrict__ gp = gr + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    const Acc ge = Cvt<Tdy, Acc>::load(gp[k]);
    sa += ge;
    sb += ge * ((Cvt<Tx, Acc>::load(xp[k]) - m) * r);
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc xe[kUnroll][8], ge[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<Tx, Acc>(xp + rs.head + 8 * j, xe[u]);
        load8<Tdy, Acc>(gp + rs.head + 8 * j, ge[u]);
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          xe[u][t] = m;
          ge[u][t] = Acc(0);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        sa += ge[u][t];
        sb += ge[u][t] * ((xe[u][t] - m) * r);
      }
  }
  double a = sa, b = sb;
  block_sum2(a, b);
  if (threadIdx.x == 0) {
    part[(ck.row * splits + ck.split) * 2] = a;
    part[(ck.row * splits + ck.split) * 2 + 1] = b;
  }
}

template <typename Tdy, typename Tx>
__global__ __launch_bounds__(kThreads) void gn_bwd_apply_kernel(
    const Tdy* __restrict__ dy, const Tx* __restrict__ x, const void* __restrict__ mean,
    const void* __restrict__ rstd, const void* __restrict__ gamma, int pdtype,
    Tx* __restrict__ dx, int64_t c, int64_t v, int splits, int64_t chunk, bool vec_ok,
    const double* __restrict__ part, double* __restrict__ rows_out, void* __restrict__ dgamma,
    void* __restrict__ dbeta) {
  using Acc = typename AccOf<Tx>::type;
  const Chunk ck = chunk_of_block(v, splits, chunk);
  double sa, sb;
  combine_row(part, ck.row, splits, sa, sb);
  if (ck.split == 0 && threadIdx.x == 0) {
    rows_out[ck.row * 2] = sa;
    rows_out[ck.row * 2 + 1] = sb;
    // One sample (dgamma / dbeta passed): the row sums are the parameter
    // gradients, stored as gn_param_grad_kernel would store them (0 + sum).
    if (dgamma) store_param(dgamma, pdtype, ck.row, 0.0 + sb);
    if (dbeta) store_param(dbeta, pdtype, ck.row, 0.0 + sa);
  }
  if (dx == nullptr) return;
  const Tx* __restrict__ xr = x + ck.row * v;
  const Tdy* __restrict__ gr = dy + ck.row * v;
  Tx* __restrict__ out = dx + ck.row * v;
  const double m = load_stat<Acc>(mean, ck.row);
  const double r = load_stat<Acc>(rstd, ck.row);
  const double g = gamma ? load_param(gamma, pdtype, ck.row % c) : 1.0;
  const double inv_n = 1.0 / static_cast<double>(v);
  // dx = r*g*(dy - A/V) - xhat * (r*g*B/V), xhat = (x - m)*r
  const Acc k1 = static_cast<Acc>(r * g);
  const Acc ma = static_cast<Acc>(sa * inv_n);
  const Acc kb = static_cast<Acc>(r * g * sb * inv_n);
  const Acc mf = static_cast<Acc>(m);
  const Acc rf = static_cast<Acc>(r);
  const Tx* __restrict__ xp = xr + ck.begin;
  const Tdy* __restrict__ gp = gr + ck.begin;
  Tx* __restrict__ op = out + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    const Acc xe = Cvt<Tx, Acc>::load(xp[k]);
    const Acc ge = Cvt<Tdy, Acc>::load(gp[k]);
    op[k] = Cvt<Tx, Acc>::store(k1 * (ge - ma) - ((xe - mf) * rf) * kb);
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc xe[kUnroll][8], ge[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<Tx, Acc>(xp + rs.head + 8 * j, xe[u]);
        load8<Tdy, Acc>(gp + rs.head + 8 * j, ge[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xe[u][t] = k1 * (ge[u][t] - ma) - ((xe[u][t] - mf) * rf) * kb;
        store8<Tx, Acc>(op + rs.head + 8 * j, xe[u]);
      }
    }
  }
}

__global__ void gn_param_grad_kernel(const double* __restrict__ rows, int64_t n, int64_t c,
                                     void* __restrict__ dgamma, void* __restrict__ dbeta,
                                     int pdtype) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double sa = 0.0, sb = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    sa += rows[(i * c + ch) * 2];
    sb += rows[(i * c + ch) * 2 + 1];
  }
  if (dgamma) store_param(dgamma, pdtype, ch, sb);
  if (dbeta) store_param(dbeta, pdtype, ch, sa);
}

// ------------------------------------------------------------------ host side

bool dtype_ok(int d) { return d >= MEDNEXT_DTYPE_F32 && d <= MEDNEXT_DTYPE_BF16; }

int64_t chunk_len(int64_t v, int splits) {
  int64_t ch = cdiv(v, splits);
  return cdiv(ch, 8) * 8;  // chunk starts stay 8-element aligned relative to the row
}

// Vector accesses assume every tensor's base is 64-byte aligned (8 elements of
// up to 8 bytes), so that global element index % 8 decides alignment.
bool aligned64(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 63u) == 0; }

size_t workspace_need(int64_t n, int64_t c, int splits) {
  return static_cast<size_t>(n * c * (static_cast<int64_t>(splits) + 1) * 2 * sizeof(double));
}

template <typename Tx, typename Ty>
int gn_fwd_typed(const void* x, const void* gamma, const void* beta, int pdtype, void* y,
                 void* mean, void* rstd, int64_t n, int64_t c, int64_t v, double eps, int splits,
                 double* part, hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  const bool vec_ok = aligned64(x) && aligned64(y);
  hipLaunchKernelGGL((gn_stats_kernel<Tx>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads),
                     0, st, static_cast<const Tx*>(x), v, splits, chunk, vec_ok, part);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL((gn_apply_kernel<Tx, Ty>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kThreads), 0, st, static_cast<const Tx*>(x), gamma, beta, pdtype,
                     static_cast<Ty*>(y), mean, rstd, c, v, eps, splits, chunk, vec_ok, part);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename Tx>
int gn_stats_typed(const void* x, const void* gamma, const void* beta, int pdtype, void* mean, void* rstd,
                   double* coef, int64_t n, int64_t c, int64_t v, double eps, int splits, double* part,
                   hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  hipLaunchKernelGGL((gn_stats_kernel<Tx>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const Tx*>(x), v, splits, chunk, aligned64(x), part);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL((gn_coef_kernel<Tx>), dim3(static_cast<unsigned>(cdiv(n * c, int64_t(256)))), dim3(256), 0, st,
                     static_cast<const Tx*>(x), gamma, beta, pdtype, mean, rstd, coef, n * c, c, v, eps, splits,
                     part);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename Tdy, typename Tx>
int gn_bwd_typed(const void* dy, const void* x, const void* mean, const void* rstd,
                 const void* gamma, int pdtype, void* dx, void* dgamma, void* dbeta, int64_t n,
                 int64_t c, int64_t v, int splits, double* part, hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  double* rows = part + n * c * splits * 2;
  const bool vec_ok = aligned64(dy) && aligned64(x) && aligned64(dx);
  hipLaunchKernelGGL((gn_bwd_reduce_kernel<Tdy, Tx>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kThreads), 0, st, static_cast<const Tdy*>(dy),
                     static_cast<const Tx*>(x), mean, rstd, v, splits, chunk, vec_ok, part);
  MEDNEXT_CHECK_LAUNCH();
  // One sample: the apply kernel stores the parameter gradients itself.
  const bool one = n == 1;
  hipLaunchKernelGGL((gn_bwd_apply_kernel<Tdy, Tx>), dim3(static_cast<unsigned>(blocks)),
                     dim3(kThreads), 0, st, static_cast<const Tdy*>(dy),
                     static_cast<const Tx*>(x), mean, rstd, gamma, pdtype, static_cast<Tx*>(dx),
                     c, v, splits, chunk, vec_ok, part, rows, one ? dgamma : nullptr, one ? dbeta : nullptr);
  MEDNEXT_CHECK_LAUNCH();
  if (!one && (dgamma || dbeta)) {
    hipLaunchKernelGGL(gn_param_grad_kernel, dim3(static_cast<unsigned>(cdiv(c, 256))),
                       dim3(256), 0, st, rows, n, c, dgamma, dbeta, pdtype);
    MEDNEXT_CHECK_LAUNCH();
  }
  return MEDNEXT_STATUS_OK;
}

int check_common(int64_t n, int64_t c, int64_t v, int splits) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && v >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(splits >= 1 && splits <= 4096, "splits must be in [1, 4096]");
  MEDNEXT_CHECK_ARG(n * c * splits < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

}  // namespace
}  // namespace mednext

using namespace mednext;

extern "C" size_t mednext_group_norm_workspace_bytes(int64_t n, int64_t c, int64_t spatial,
                                                     int32_t splits) {
  (void)spatial;
  if (n < 1 || c < 1 || splits < 1) return 0;
  return workspace_need(n, c, splits);
}

extern "C" int32_t mednext_group_norm_fwd(const void* x, int32_t x_dtype, const void* gamma,
                                          const void* beta, int32_t param_dtype, void* y,
                                          int32_t y_dtype, void* mean, void* rstd, int64_t n,
                                          int64_t c, int64_t spatial, double eps, int32_t splits,
                                          void* workspace, size_t workspace_bytes,
                                          void* stream) {
  int st = check_common(n, c, spatial, splits);
  if (st) return st;
  MEDNEXT_CHECK_ARG(x && y && mean && rstd, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(y_dtype) && dtype_ok(param_dtype),
                    "unsupported dtype");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= workspace_need(n, c, splits),
                    "workspace too small");
  MEDNEXT_CHECK_ARG(eps >= 0.0, "eps must be non-negative");
  auto part = static_cast<double*>(workspace);
  auto s = static_cast<hipStream_t>(stream);
#define GN_FWD(TX, TY) \
  gn_fwd_typed<TX, TY>(x, gamma, beta, param_dtype, y, mean, rstd, n, c, spatial, eps, splits, part, s)
  if (x_dtype == MEDNEXT_DTYPE_F64 && y_dtype == MEDNEXT_DTYPE_F64) return GN_FWD(double, double);
  if (x_dtype == MEDNEXT_DTYPE_F32 && y_dtype == MEDNEXT_DTYPE_F32) return GN_FWD(float, float);
  if (x_dtype == MEDNEXT_DTYPE_BF16 && y_dtype == MEDNEXT_DTYPE_F32) return GN_FWD(bf16_t, float);
  if (x_dtype == MEDNEXT_DTYPE_BF16 && y_dtype == MEDNEXT_DTYPE_BF16) return GN_FWD(bf16_t, bf16_t);
  if (x_dtype == MEDNEXT_DTYPE_F16 && y_dtype == MEDNEXT_DTYPE_F32) return GN_FWD(f16_t, float);
  if (x_dtype == MEDNEXT_DTYPE_F16 && y_dtype == MEDNEXT_DTYPE_F16) return GN_FWD(f16_t, f16_t);
#undef GN_FWD
  set_error("mednext_group_norm_fwd: unsupported (x, y) dtype pair");
  return MEDNEXT_STATUS_UNSUPPORTED;
}

extern "C" int32_t mednext_group_norm_stats(const void* x, int32_t x_dtype, const void* gamma,
                                            const void* beta, int32_t param_dtype, void* mean, void* rstd,
                                            void* coef, int64_t n, int64_t c, int64_t spatial, double eps,
                                            int32_t splits, void* workspace, size_t workspace_bytes,
                                            void* stream) {
  int st = check_common(n, c, spatial, splits);
  if (st) return st;
  MEDNEXT_CHECK_ARG(x && mean && rstd && coef, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(param_dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG((reinterpret_cast<uintptr_t>(coef) & 7u) == 0, "coef must be 8-byte aligned");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= workspace_need(n, c, splits), "workspace too small");
  MEDNEXT_CHECK_ARG(eps >= 0.0, "eps must be non-negative");
  auto part = static_cast<double*>(workspace);
  auto s = static_cast<hipStream_t>(stream);
  auto cf = static_cast<double*>(coef);
  switch (x_dtype) {
    case MEDNEXT_DTYPE_F64:
      return gn_stats_typed<double>(x, gamma, beta, param_dtype, mean, rstd, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F32:
      return gn_stats_typed<float>(x, gamma, beta, param_dtype, mean, rstd, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F16:
      return gn_stats_typed<f16_t>(x, gamma, beta, param_dtype, mean, rstd, cf, n, c, spatial, eps, splits, part, s);
    default:
      return gn_stats_typed<bf16_t>(x, gamma, beta, param_dtype, mean, rstd, cf, n, c, spatial, eps, splits, part,
                                    s);
  }
}

extern "C" int32_t mednext_group_norm_bwd(const void* grad_output, int32_t dy_dtype, const void* x,
                                          int32_t x_dtype, const void* mean, const void* rstd,
                                          const void* gamma, int32_t param_dtype,
                                          void* grad_input, void* grad_gamma, void* grad_beta,
                                          int64_t n, int64_t c, int64_t spatial, int32_t splits,
                                          void* workspace, size_t workspace_bytes,
                                          void* stream) {
  int st = check_common(n, c, spatial, splits);
  if (st) return st;
  MEDNEXT_CHECK_ARG(grad_output && x && mean && rstd, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(dy_dtype) && dtype_ok(param_dtype),
                    "unsupported dtype");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= workspace_need(n, c, splits),
                    "workspace too small");
  auto part = static_cast<double*>(workspace);
  auto s = static_cast<hipStream_t>(stream);
#define GN_BWD(TDY, TX)                                                                        \
  gn_bwd_typed<TDY, TX>(grad_output, x, mean, rstd, gamma, param_dtype, grad_input, grad_gamma, \
                        grad_beta, n, c, spatial, splits, part, s)
  if (dy_dtype == MEDNEXT_DTYPE_F64 && x_dtype == MEDNEXT_DTYPE_F64) return GN_BWD(double, double);
  if (dy_dtype == MEDNEXT_DTYPE_F32 && x_dtype == MEDNEXT_DTYPE_F32) return GN_BWD(float, float);
  if (dy_dtype == MEDNEXT_DTYPE_F32 && x_dtype == MEDNEXT_DTYPE_BF16) return GN_BWD(float, bf16_t);
  if (dy_dtype == MEDNEXT_DTYPE_BF16 && x_dtype == MEDNEXT_DTYPE_BF16) return GN_BWD(bf16_t, bf16_t);
  if (dy_dtype == MEDNEXT_DTYPE_F32 && x_dtype == MEDNEXT_DTYPE_F16) return GN_BWD(float, f16_t);
  if (dy_dtype == MEDNEXT_DTYPE_F16 && x_dtype == MEDNEXT_DTYPE_F16) return GN_BWD(f16_t, f16_t);
#undef GN_BWD
  set_error("mednext_group_norm_bwd: unsupported (grad_output, x) dtype pair");
  return MEDNEXT_STATUS_UNSUPPORTED;
}
