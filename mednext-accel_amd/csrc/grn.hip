// Global Response Normalization over NCDHW (MedNeXt v2), forward and backward,
// for gfx950. Per sample n and channel c, with x_c the channel's voxels:
//   n_c = ||x_c||_2,  S = sum_c n_c,  r_c = n_c / (S + eps)
//   y   = x + gamma_c * x * r_c + beta_c = x * (1 + gamma_c r_c) + beta_c
// computed in fp32 from any input dtype (fp64 for fp64) and stored in the
// input dtype. Backward, with g_c = sum_v dy x and T = sum_c gamma_c g_c n_c:
//   dx = dy (1 + gamma_c r_c) + x (gamma_c g_c / (S + eps) - T / (S + eps)^2) / n_c
//   dgamma_c = sum_n g_c r_c,  dbeta_c = sum_n sum_v dy
// (the x / n_c term is taken as zero where n_c == 0, the subgradient the
// reference's vector norm uses).
//
// Three launches each way: (1) per-(n, c) row chunks reduce sum x^2 (forward)
// or sum dy x and sum dy (backward) into fp64 partials, one workgroup per
// chunk; (2) one workgroup per sample combines the partials in a fixed order
// and derives the per-(n, c) coefficients; (3) an elementwise pass applies
// them. Rows stream as a scalar head, 16-byte vectors and a scalar tail, so any
// volume is handled. All reductions are fixed-order (bit-reproducible).
#include "common.h"

namespace mednext {
namespace {

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

struct Chunk {
  int64_t row;  // n * C + c
  int split;
  int64_t begin, end;
};

__device__ inline Chunk chunk_of(int64_t v, int splits, int64_t chunk) {
  Chunk ck;
  ck.row = blockIdx.x / splits;
  ck.split = static_cast<int>(blockIdx.x % splits);
  ck.begin = static_cast<int64_t>(ck.split) * chunk;
  ck.end = ck.begin + chunk < v ? ck.begin + chunk : v;
  return ck;
}

// Fixed-order block sum of two doubles; valid in thread 0.
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
    for (int w = 1; w < kThreads / 64; ++w) {
      a += red[w][0];
      b += red[w][1];
    }
  }
}

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

// Pass 1 (forward): partial sum of squares per (row, split).
template <typename T>
__global__ __launch_bounds__(kThreads) void grn_sumsq_kernel(const T* __restrict__ x, int64_t v, int splits,
                                                            int64_t chunk, bool vec_ok, double* __restrict__ part) {
  using Acc = typename AccOf<T>::type;
  const Chunk ck = chunk_of(v, splits, chunk);
  const T* __restrict__ cp = x + ck.row * v + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  Acc s = Acc(0);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const Acc e = Cvt<T, Acc>::load(cp[rs.scalar_index(i)]);
    s += e * e;
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc e[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<T, Acc>(cp + rs.head + 8 * j, e[u]);
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) e[u][t] = Acc(0);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 8; ++t) s += e[u][t] * e[u][t];
  }
  double a = s, b = 0.0;
  block_sum2(a, b);
  if (threadIdx.x == 0) part[ck.row * splits + ck.split] = a;
}

// Pass 2 (forward): one workgroup per sample. coef[row] = (1 + gamma r, beta, r, n).
__global__ __launch_bounds__(kThreads) void grn_fwd_coef_kernel(const double* __restrict__ part, int64_t c,
                                                               int splits, const void* __restrict__ gamma,
                                                               const void* __restrict__ beta, int pdtype,
                                                               double eps, double* __restrict__ coef) {
  const int64_t n = blockIdx.x;
  __shared__ double norms_sum;
  // Norms in fixed order: each thread owns channels tid, tid + 256, ...
  double local = 0.0;
  for (int64_t ch = threadIdx.x; ch < c; ch += blockDim.x) {
    const double* p = part + (n * c + ch) * splits;
    double sq = 0.0;
    for (int s = 0; s < splits; ++s) sq += p[s];
    const double nrm = sqrt(sq);
    coef[(n * c + ch) * 4 + 3] = nrm;
    local += nrm;
  }
  double dummy = 0.0;
  block_sum2(local, dummy);
  if (threadIdx.x == 0) norms_sum = local;
  __syncthreads();
  const double denom = norms_sum + eps;
  for (int64_t ch = threadIdx.x; ch < c; ch += blockDim.x) {
    double* cf = coef + (n * c + ch) * 4;
    const double r = cf[3] / denom;
    const double g = gamma ? load_param(gamma, pdtype, ch) : 0.0;
    const double b = beta ? load_param(beta, pdtype, ch) : 0.0;
    cf[0] = 1.0 + g * r;
    cf[1] = b;
    cf[2] = r;
  }
}

// Pass 3 (forward): y = x * scale + shift.
template <typename T>
__global__ __launch_bounds__(kThreads) void grn_apply_kernel(const T* __restrict__ x, T* __restrict__ y, int64_t v,
                                                            int splits, int64_t chunk, bool vec_ok,
                                                            const double* __restrict__ coef) {
  using Acc = typename AccOf<T>::type;
  const Chunk ck = chunk_of(v, splits, chunk);
  const Acc scale = static_cast<Acc>(coef[ck.row * 4]);
  const Acc shift = static_cast<Acc>(coef[ck.row * 4 + 1]);
  const T* __restrict__ cp = x + ck.row * v + ck.begin;
  T* __restrict__ op = y + ck.row * v + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    op[k] = Cvt<T, Acc>::store(Cvt<T, Acc>::load(cp[k]) * scale + shift);
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc e[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) load8<T, Acc>(cp + rs.head + 8 * j, e[u]);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
#pragma unroll
        for (int t = 0; t < 8; ++t) e[u][t] = e[u][t] * scale + shift;
        store8<T, Acc>(op + rs.head + 8 * j, e[u]);
      }
    }
  }
}

// Pass 1 (backward): partial (sum dy x, sum dy) per (row, split).
template <typename Tdy, typename T>
__global__ __launch_bounds__(kThreads) void grn_bwd_reduce_kernel(const Tdy* __restrict__ dy, const T* __restrict__ x,
                                                                 int64_t v, int splits, int64_t chunk, bool vec_ok,
                                                                 double* __restrict__ part) {
  using Acc = typename AccOf<T>::type;
  const Chunk ck = chunk_of(v, splits, chunk);
  const T* __restrict__ xp = x + ck.row * v + ck.begin;
  const Tdy* __restrict__ gp = dy + ck.row * v + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  Acc sg = Acc(0), sd = Acc(0);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    const Acc ge = Cvt<Tdy, Acc>::load(gp[k]);
    sg += ge * Cvt<T, Acc>::load(xp[k]);
    sd += ge;
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc xe[kUnroll][8], ge[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<T, Acc>(xp + rs.head + 8 * j, xe[u]);
        load8<Tdy, Acc>(gp + rs.head + 8 * j, ge[u]);
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t) xe[u][t] = ge[u][t] = Acc(0);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        sg += ge[u][t] * xe[u][t];
        sd += ge[u][t];
      }
  }
  double a = sg, b = sd;
  block_sum2(a, b);
  if (threadIdx.x == 0) {
    part[(ck.row * splits + ck.split) * 2] = a;
    part[(ck.row * splits + ck.split) * 2 + 1] = b;
  }
}

// Pass 2 (backward): one workgroup per sample. From the forward's saved
// (n_c, r_c) and the reduced (g_c, sum dy): k1 = 1 + gamma r, k2 = (gamma g /
// (S + eps) - T / (S + eps)^2) / n_c, and the per-sample parameter-gradient
// terms rows[(n, c)] = (g_c r_c, sum dy).
__global__ __launch_bounds__(kThreads) void grn_bwd_coef_kernel(const double* __restrict__ part,
                                                               const double* __restrict__ fcoef, int64_t c,
                                                               int splits, const void* __restrict__ gamma, int pdtype,
                                                               double eps, double* __restrict__ bcoef,
                                                               double* __restrict__ rows) {
  const int64_t n = blockIdx.x;
  __shared__ double totals[2];
  double s_norm = 0.0, t_sum = 0.0;
  for (int64_t ch = threadIdx.x; ch < c; ch += blockDim.x) {
    const double* p = part + (n * c + ch) * splits * 2;
    double g = 0.0, sd = 0.0;
    for (int s = 0; s < splits; ++s) {
      g += p[2 * s];
      sd += p[2 * s + 1];
    }
    const double* fc = fcoef + (n * c + ch) * 4;
    const double gam = gamma ? load_param(gamma, pdtype, ch) : 0.0;
    s_norm += fc[3];
    t_sum += gam * g * fc[3];
    rows[(n * c + ch) * 2] = g * fc[2];
    rows[(n * c + ch) * 2 + 1] = sd;
    bcoef[(n * c + ch) * 2 + 1] = gam * g;  // stashed, finished below
  }
  block_sum2(s_norm, t_sum);
  if (threadIdx.x == 0) {
    totals[0] = s_norm;
    totals[1] = t_sum;
  }
  __syncthreads();
  const double denom = totals[0] + eps;
  const double t_term = totals[1] / (denom * denom);
  for (int64_t ch = threadIdx.x; ch < c; ch += blockDim.x) {
    const double* fc = fcoef + (n * c + ch) * 4;
    double* bc = bcoef + (n * c + ch) * 2;
    const double gam = gamma ? load_param(gamma, pdtype, ch) : 0.0;
    const double nrm = fc[3];
    bc[0] = 1.0 + gam * fc[2];
    bc[1] = nrm > 0.0 ? (bc[1] / denom - t_term) / nrm : 0.0;
  }
}

// Pass 3 (backward): dx = dy * k1 + x * k2.
template <typename Tdy, typename T>
__global__ __launch_bounds__(kThreads) void grn_bwd_apply_kernel(const Tdy* __restrict__ dy, const T* __restrict__ x,
                                                                T* __restrict__ dx, int64_t v, int splits,
                                                                int64_t chunk, bool vec_ok,
                                                                const double* __restrict__ bcoef) {
  using Acc = typename AccOf<T>::type;
  const Chunk ck = chunk_of(v, splits, chunk);
  const Acc k1 = static_cast<Acc>(bcoef[ck.row * 2]);
  const Acc k2 = static_cast<Acc>(bcoef[ck.row * 2 + 1]);
  const T* __restrict__ xp = x + ck.row * v + ck.begin;
  const Tdy* __restrict__ gp = dy + ck.row * v + ck.begin;
  T* __restrict__ op = dx + ck.row * v + ck.begin;
  const RowSpan rs = row_span(ck.row * v + ck.begin, ck.end - ck.begin, vec_ok);
  for (int64_t i = threadIdx.x; i < rs.scalar_count(); i += blockDim.x) {
    const int64_t k = rs.scalar_index(i);
    op[k] = Cvt<T, Acc>::store(Cvt<Tdy, Acc>::load(gp[k]) * k1 + Cvt<T, Acc>::load(xp[k]) * k2);
  }
  for (int64_t j0 = threadIdx.x; j0 < rs.nvec; j0 += kUnroll * blockDim.x) {
    Acc xe[kUnroll][8], ge[kUnroll][8];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
        load8<T, Acc>(xp + rs.head + 8 * j, xe[u]);
        load8<Tdy, Acc>(gp + rs.head + 8 * j, ge[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t j = j0 + u * static_cast<int64_t>(blockDim.x);
      if (j < rs.nvec) {
#pragma unroll
        for (int t = 0; t < 8; ++t) xe[u][t] = ge[u][t] * k1 + xe[u][t] * k2;
        store8<T, Acc>(op + rs.head + 8 * j, xe[u]);
      }
    }
  }
}

// Row sums of GEMM-epilogue partials: one wave per (n, c) row; lane l sums
// slots l, l + 64, ... in order, then a fixed wave reduction.
__global__ __launch_bounds__(64) void grn_row_sum_kernel(const double* __restrict__ rpart, int64_t slots,
                                                       double* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const double* p = rpart + row * slots * 2;
  double a = 0.0, b = 0.0;
  for (int64_t s = threadIdx.x; s < slots; s += 64) {
    a += p[2 * s];
    b += p[2 * s + 1];
  }
  a = wave_sum(a);
  b = wave_sum(b);
  if (threadIdx.x == 0) {
    out[row * 2] = a;
    out[row * 2 + 1] = b;
  }
}

__global__ void grn_param_grad_kernel(const double* __restrict__ rows, int64_t n, int64_t c,
                                      void* __restrict__ dgamma, void* __restrict__ dbeta, int pdtype) {
  const int64_t ch = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (ch >= c) return;
  double sg = 0.0, sb = 0.0;
  for (int64_t i = 0; i < n; ++i) {
    sg += rows[(i * c + ch) * 2];
    sb += rows[(i * c + ch) * 2 + 1];
  }
  if (dgamma) store_param(dgamma, pdtype, ch, sg);
  if (dbeta) store_param(dbeta, pdtype, ch, sb);
}

// ------------------------------------------------------------------ host side

bool dtype_ok(int d) { return d >= MEDNEXT_DTYPE_F32 && d <= MEDNEXT_DTYPE_BF16; }
bool aligned64(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 63u) == 0; }
int64_t chunk_len(int64_t v, int splits) { return cdiv(cdiv(v, splits), 8) * 8; }

int check_shape(int64_t n, int64_t c, int64_t v, int splits) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1 && v >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(splits >= 1 && splits <= 4096, "splits must be in [1, 4096]");
  MEDNEXT_CHECK_ARG(n * c * splits < (int64_t(1) << 31) && n < (int64_t(1) << 31), "grid too large");
  return MEDNEXT_STATUS_OK;
}

// Forward workspace: fp64 partial sums [N*C*splits].
size_t fwd_workspace(int64_t n, int64_t c, int splits) { return static_cast<size_t>(n * c * splits) * sizeof(double); }
// Backward workspace: partials [N*C*splits*2] + coefficients [N*C*2] + rows [N*C*2].
size_t bwd_workspace(int64_t n, int64_t c, int splits) {
  return static_cast<size_t>(n * c * (static_cast<int64_t>(splits) * 2 + 4)) * sizeof(double);
}

// Pass 1 + pass 2 only: coef without an output tensor.
template <typename T>
int grn_stats_typed(const void* x, const void* gamma, const void* beta, int pdtype, double* coef, int64_t n,
                    int64_t c, int64_t v, double eps, int splits, double* part, hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  hipLaunchKernelGGL((grn_sumsq_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const T*>(x), v, splits, chunk, aligned64(x), part);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL(grn_fwd_coef_kernel, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, part, c, splits,
                     gamma, beta, pdtype, eps, coef);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename T>
int grn_fwd_typed(const void* x, const void* gamma, const void* beta, int pdtype, void* y, double* coef, int64_t n,
                  int64_t c, int64_t v, double eps, int splits, double* part, hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  const bool vec_ok = aligned64(x) && aligned64(y);
  hipLaunchKernelGGL((grn_sumsq_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const T*>(x), v, splits, chunk, vec_ok, part);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL(grn_fwd_coef_kernel, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, part, c, splits,
                     gamma, beta, pdtype, eps, coef);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL((grn_apply_kernel<T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const T*>(x), static_cast<T*>(y), v, splits, chunk, vec_ok, coef);
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

template <typename Tdy, typename T>
int grn_bwd_typed(const void* dy, const void* x, const double* coef, const void* gamma, int pdtype, void* dx,
                  void* dgamma, void* dbeta, int64_t n, int64_t c, int64_t v, double eps, int splits, double* ws,
                  hipStream_t st) {
  const int64_t chunk = chunk_len(v, splits);
  const int64_t blocks = n * c * splits;
  double* part = ws;
  double* bcoef = part + n * c * splits * 2;
  double* rows = bcoef + n * c * 2;
  const bool vec_ok = aligned64(dy) && aligned64(x) && aligned64(dx);
  hipLaunchKernelGGL((grn_bwd_reduce_kernel<Tdy, T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                     static_cast<const Tdy*>(dy), static_cast<const T*>(x), v, splits, chunk, vec_ok, part);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL(grn_bwd_coef_kernel, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, st, part, coef, c,
                     splits, gamma, pdtype, eps, bcoef, rows);
  MEDNEXT_CHECK_LAUNCH();
  if (dx != nullptr) {
    hipLaunchKernelGGL((grn_bwd_apply_kernel<Tdy, T>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, st,
                       static_cast<const Tdy*>(dy), static_cast<const T*>(x), static_cast<T*>(dx), v, splits, chunk,
                       vec_ok, bcoef);
    MEDNEXT_CHECK_LAUNCH();
  }
  if (dgamma || dbeta) {
    hipLaunchKernelGGL(grn_param_grad_kernel, dim3(static_cast<unsigned>(cdiv(c, 256))), dim3(256), 0, st, rows, n,
                       c, dgamma, dbeta, pdtype);
    MEDNEXT_CHECK_LAUNCH();
  }
  return MEDNEXT_STATUS_OK;
}

}  // namespace
}  // namespace mednext

using namespace mednext;

extern "C" size_t mednext_grn_workspace_bytes(int64_t n, int64_t c, int64_t spatial, int32_t splits) {
  (void)spatial;
  if (n < 1 || c < 1 || splits < 1) return 0;
  return bwd_workspace(n, c, splits) > fwd_workspace(n, c, splits) ? bwd_workspace(n, c, splits)
                                                                     : fwd_workspace(n, c, splits);
}

extern "C" int32_t mednext_grn_fwd(const void* x, int32_t x_dtype, const void* gamma, const void* beta,
                                   int32_t param_dtype, void* y, void* coef, int64_t n, int64_t c, int64_t spatial,
                                   double eps, int32_t splits, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (int st = check_shape(n, c, spatial, splits)) return st;
  MEDNEXT_CHECK_ARG(x && y && coef, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(param_dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(eps > 0.0, "eps must be positive");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= fwd_workspace(n, c, splits), "workspace too small");
  auto* part = static_cast<double*>(workspace);
  auto* cf = static_cast<double*>(coef);
  auto s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case MEDNEXT_DTYPE_F32: return grn_fwd_typed<float>(x, gamma, beta, param_dtype, y, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F64: return grn_fwd_typed<double>(x, gamma, beta, param_dtype, y, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F16: return grn_fwd_typed<f16_t>(x, gamma, beta, param_dtype, y, cf, n, c, spatial, eps, splits, part, s);
    default: return grn_fwd_typed<bf16_t>(x, gamma, beta, param_dtype, y, cf, n, c, spatial, eps, splits, part, s);
  }
}

extern "C" int32_t mednext_grn_bwd(const void* grad_output, int32_t dy_dtype, const void* x, int32_t x_dtype,
                                   const void* coef, const void* gamma, int32_t param_dtype, void* grad_input,
                                   void* grad_gamma, void* grad_beta, int64_t n, int64_t c, int64_t spatial,
                                   double eps, int32_t splits, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  if (int st = check_shape(n, c, spatial, splits)) return st;
  MEDNEXT_CHECK_ARG(grad_output && x && coef, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(dy_dtype) && dtype_ok(param_dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(eps > 0.0, "eps must be positive");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= bwd_workspace(n, c, splits), "workspace too small");
  auto* ws = static_cast<double*>(workspace);
  const auto* cf = static_cast<const double*>(coef);
  auto s = static_cast<hipStream_t>(stream);
#define GRN_BWD(TDY, TX) \
  grn_bwd_typed<TDY, TX>(grad_output, x, cf, gamma, param_dtype, grad_input, grad_gamma, grad_beta, n, c, spatial, eps, splits, ws, s)
  if (dy_dtype == x_dtype) {
    switch (x_dtype) {
      case MEDNEXT_DTYPE_F32: return GRN_BWD(float, float);
      case MEDNEXT_DTYPE_F64: return GRN_BWD(double, double);
      case MEDNEXT_DTYPE_F16: return GRN_BWD(f16_t, f16_t);
      default: return GRN_BWD(bf16_t, bf16_t);
    }
  }
  if (dy_dtype == MEDNEXT_DTYPE_F32 && x_dtype == MEDNEXT_DTYPE_BF16) return GRN_BWD(float, bf16_t);
  if (dy_dtype == MEDNEXT_DTYPE_F32 && x_dtype == MEDNEXT_DTYPE_F16) return GRN_BWD(float, f16_t);
#undef GRN_BWD
  set_error("mednext_grn_bwd: unsupported (grad_output, x) dtype pair");
  return MEDNEXT_STATUS_UNSUPPORTED;
}

extern "C" int32_t mednext_grn_stats(const void* x, int32_t x_dtype, const void* gamma,
                                     const void* beta, int32_t param_dtype, void* coef, int64_t n, int64_t c,
                                     int64_t spatial, double eps, int32_t splits, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (int st = check_shape(n, c, spatial, splits)) return st;
  MEDNEXT_CHECK_ARG(x && coef, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(x_dtype) && dtype_ok(param_dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(eps > 0.0, "eps must be positive");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= fwd_workspace(n, c, splits), "workspace too small");
  auto* part = static_cast<double*>(workspace);
  auto* cf = static_cast<double*>(coef);
  auto s = static_cast<hipStream_t>(stream);
  switch (x_dtype) {
    case MEDNEXT_DTYPE_F32: return grn_stats_typed<float>(x, gamma, beta, param_dtype, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F64: return grn_stats_typed<double>(x, gamma, beta, param_dtype, cf, n, c, spatial, eps, splits, part, s);
    case MEDNEXT_DTYPE_F16: return grn_stats_typed<f16_t>(x, gamma, beta, param_dtype, cf, n, c, spatial, eps, splits, part, s);
    default: return grn_stats_typed<bf16_t>(x, gamma, beta, param_dtype, cf, n, c, spatial, eps, splits, part, s);
  }
}

extern "C" int32_t mednext_grn_bwd_rows(const void* row_partial, int64_t slots, const void* coef,
                                        const void* gamma, int32_t param_dtype, void* coef_out, void* grad_gamma,
                                        void* grad_beta, int64_t n, int64_t c, double eps, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1, "shape must be positive");
  MEDNEXT_CHECK_ARG(slots >= 1 && slots < (int64_t(1) << 24), "slots must be in [1, 2^24)");
  MEDNEXT_CHECK_ARG(n < (int64_t(1) << 31) && n * c * slots < (int64_t(1) << 40), "problem too large");
  MEDNEXT_CHECK_ARG(row_partial && coef && coef_out, "null tensor pointer");
  MEDNEXT_CHECK_ARG(dtype_ok(param_dtype), "unsupported dtype");
  MEDNEXT_CHECK_ARG(eps > 0.0, "eps must be positive");
  MEDNEXT_CHECK_ARG(workspace && workspace_bytes >= static_cast<size_t>(n * c * 4) * sizeof(double),
                    "workspace too small");
  MEDNEXT_CHECK_ARG(n * c < (int64_t(1) << 31), "grid too large");
  auto s = static_cast<hipStream_t>(stream);
  auto* sums = static_cast<double*>(workspace);
  double* rows = sums + n * c * 2;
  hipLaunchKernelGGL(grn_row_sum_kernel, dim3(static_cast<unsigned>(n * c)), dim3(64), 0, s,
                     static_cast<const double*>(row_partial), slots, sums);
  MEDNEXT_CHECK_LAUNCH();
  hipLaunchKernelGGL(grn_bwd_coef_kernel, dim3(static_cast<unsigned>(n)), dim3(kThreads), 0, s, sums,
                     static_cast<const double*>(coef), c, 1, gamma, param_dtype, eps, static_cast<double*>(coef_out),
                     rows);
  MEDNEXT_CHECK_LAUNCH();
  if (grad_gamma || grad_beta) {
    hipLaunchKernelGGL(grn_param_grad_kernel, dim3(static_cast<unsigned>(cdiv(c, 256))), dim3(256), 0, s, rows, n,
                       c, grad_gamma, grad_beta, param_dtype);
    MEDNEXT_CHECK_LAUNCH();
  }
  return MEDNEXT_STATUS_OK;
}
