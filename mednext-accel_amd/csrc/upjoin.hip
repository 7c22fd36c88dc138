// The tail of a MedNeXt up block in one pass each way (bf16).
//
// The up block's main branch ends at (2s - 1)^3 voxels (a stride-2
// transposed depthwise conv and the block's expansion), its residual is a
// stride-2 transposed 1x1x1 conv with bias (non-zero only at even positions
// of the same (2s - 1)^3 grid, the bias elsewhere), and both are padded by
// one voxel per dimension to (2s)^3 before they are added: at the start for
// MedNeXt v1 (reference models/blocks.py:176-181), at the end for v2
// (reference models/blocks_v2.py:128-133). With y = W^T x + b
// the residual GEMM at s^3 voxels (pointwise.hip, weight_layout 1):
//
//   out[Z][Y][X] = main[z][y][x] + (z, y, x all even ? y[z/2][y/2][x/2] : b),
//   (z, y, x) = (Z, Y, X) - lead inside the (2s - 1)^3 grid, 0 on the pad,
//
// rounded once to bf16: the value of pad(main) + pad(residual) on the same
// bf16 operands. The backward reads grad_out once and writes
//   grad_main = grad_out on the grid, grad_y = grad_out at all-even grid
//   points, grad_b = sum of grad_out over the other grid points
// (the bias at all-even points reaches y through the GEMM's own bias), or,
// with bias_over_grid, over the whole (2s - 1)^3 grid: the caller then gave
// the GEMM the bias's value only, and this sum, rounded once, is the bias's
// whole gradient, as the transposed conv's own bias reduction is. The bias
// sums are per-(n, c, plane) fp32 partials reduced in a fixed order in fp64
// by a second kernel.
//
// One workgroup per output plane (n, c, Z); each thread produces 8
// consecutive X of one row (a 16-byte store), reading main and y with element
// loads (their rows are one element shorter / half as long).
#include "cdna4.h"
#include "common.h"

namespace mednext {
namespace {

constexpr int kThreads = 256;

struct JoinGeom {
  int C, D, H, W;  // output extents (even)
  int lead;        // 1: pad at the start (v1), 0: at the end (v2)
  int bias_over_grid;  // backward: bias sum over every grid point
};

__device__ inline float ld(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }

__global__ __launch_bounds__(kThreads) void up_join_fwd_kernel(const uint16_t* __restrict__ main_in,
                                                               const uint16_t* __restrict__ small,
                                                               const uint16_t* __restrict__ bias,
                                                               uint16_t* __restrict__ out, JoinGeom g) {
  const int64_t plane = blockIdx.x;  // (n * C + c) * D + Z
  const int Z = static_cast<int>(plane % g.D);
  const int64_t nc = plane / g.D;
  const int c = static_cast<int>(nc % g.C);
  const int Dm = g.D - 1, Hm = g.H - 1, Wm = g.W - 1;  // main grid
  const int Ds = g.D / 2, Hs = g.H / 2, Ws = g.W / 2;  // residual GEMM grid
  const float b = bias != nullptr ? ld(bias, c) : 0.f;
  const int z = Z - g.lead;
  const bool zin = z >= 0 && z < Dm;
  const uint16_t* mplane = main_in + (nc * Dm + (zin ? z : 0)) * static_cast<int64_t>(Hm) * Wm;
  const uint16_t* splane = small + (nc * Ds + (zin ? z / 2 : 0)) * static_cast<int64_t>(Hs) * Ws;
  uint16_t* oplane = out + plane * static_cast<int64_t>(g.H) * g.W;
  const int groups = g.W / 8;  // W % 8 == 0 (host check)
  for (int e = threadIdx.x; e < g.H * groups; e += kThreads) {
    const int Y = e / groups, X0 = (e - Y * groups) * 8;
    const int y = Y - g.lead;
    const bool row = zin && y >= 0 && y < Hm;
    const bool even_row = row && (z % 2 == 0) && (y % 2 == 0);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int x = X0 + j - g.lead;
      float r = 0.f;
      if (row && x >= 0 && x < Wm) {
        r = ld(mplane, static_cast<int64_t>(y) * Wm + x);
        r += (even_row && x % 2 == 0) ? ld(splane, static_cast<int64_t>(y / 2) * Ws + x / 2) : b;
      }
      v[j] = r;
    }
    const uint4 o = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                               pack_bf16x2(v[6], v[7]));
    *reinterpret_cast<uint4*>(oplane + static_cast<int64_t>(Y) * g.W + X0) = o;
  }
}

__global__ __launch_bounds__(kThreads) void up_join_bwd_kernel(const uint16_t* __restrict__ dout,
                                                               uint16_t* __restrict__ dmain,
                                                               uint16_t* __restrict__ dsmall,
                                                               float* __restrict__ bias_part, JoinGeom g) {
  const int64_t plane = blockIdx.x;
  const int Z = static_cast<int>(plane % g.D);
  const int64_t nc = plane / g.D;
  const int Dm = g.D - 1, Hm = g.H - 1, Wm = g.W - 1;
  const int Ds = g.D / 2, Hs = g.H / 2, Ws = g.W / 2;
  const int z = Z - g.lead;
  const bool zin = z >= 0 && z < Dm;
  const uint16_t* gplane = dout + plane * static_cast<int64_t>(g.H) * g.W;
  uint16_t* mplane = dmain + (nc * Dm + (zin ? z : 0)) * static_cast<int64_t>(Hm) * Wm;
  uint16_t* splane = dsmall + (nc * Ds + (zin ? z / 2 : 0)) * static_cast<int64_t>(Hs) * Ws;
  float bsum = 0.f;
  if (zin) {
    const int groups = g.W / 8;
    for (int e = threadIdx.x; e < g.H * groups; e += kThreads) {
      const int Y = e / groups, X0 = (e - Y * groups) * 8;
      const int y = Y - g.lead;
      if (y < 0 || y >= Hm) continue;
      const bool even_row = (z % 2 == 0) && (y % 2 == 0);
      const uint4 gv = *reinterpret_cast<const uint4*>(gplane + static_cast<int64_t>(Y) * g.W + X0);
      const uint32_t w[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int x = X0 + j - g.lead;
        if (x < 0 || x >= Wm) continue;
        const uint16_t bits = static_cast<uint16_t>(w[j / 2] >> (16 * (j & 1)));
        mplane[static_cast<int64_t>(y) * Wm + x] = bits;
        if (even_row && x % 2 == 0) {
          splane[static_cast<int64_t>(y / 2) * Ws + x / 2] = bits;
          if (g.bias_over_grid) bsum += bf16_to_f32(bits);
        } else {
          bsum += bf16_to_f32(bits);
        }
      }
    }
  }
  // Fixed-order workgroup sum: waves, then wave 0 over the four wave totals.
  __shared__ float part[kThreads / 64];
  bsum = wave_sum(bsum);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = bsum;
  __syncthreads();
  if (threadIdx.x == 0) bias_part[plane] = (part[0] + part[1]) + (part[2] + part[3]);
}

// grad_b[c] = sum over n and planes of the partials, fp64 in a fixed order.
__global__ __launch_bounds__(64) void up_join_bias_kernel(const float* __restrict__ bias_part,
                                                          uint16_t* __restrict__ dbias, int64_t n, JoinGeom g) {
  const int c = blockIdx.x;
  double s = 0.0;
  for (int64_t i = threadIdx.x; i < n * g.D; i += 64) {
    const int64_t nn = i / g.D, Z = i - nn * g.D;
    s += static_cast<double>(bias_part[(nn * g.C + c) * g.D + Z]);
  }
  s = wave_sum(s);
  if (threadIdx.x == 0) dbias[c] = f32_to_bf16(static_cast<float>(s));
}

int check_join(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int32_t lead, int32_t dtype) {
  MEDNEXT_CHECK_ARG(dtype == MEDNEXT_DTYPE_BF16, "the up-block join takes bfloat16 tensors");
  MEDNEXT_CHECK_ARG(n >= 1 && c >= 1, "empty batch or channels");
  MEDNEXT_CHECK_ARG(d >= 2 && h >= 2 && w >= 8 && d % 2 == 0 && h % 2 == 0 && w % 8 == 0,
                    "output extents must be even, W a multiple of 8");
  MEDNEXT_CHECK_ARG(lead == 0 || lead == 1, "lead must be 0 (pad at the end) or 1 (pad at the start)");
  MEDNEXT_CHECK_ARG(n * c * d < (int64_t{1} << 31) && h * w < (int64_t{1} << 31) && c < (int64_t{1} << 31),
                    "shape too large");
  return MEDNEXT_STATUS_OK;
}

JoinGeom make_join(int64_t c, int64_t d, int64_t h, int64_t w, int32_t lead, int32_t bias_over_grid = 0) {
  return JoinGeom{static_cast<int>(c), static_cast<int>(d), static_cast<int>(h), static_cast<int>(w), lead,
                  bias_over_grid != 0 ? 1 : 0};
}

}  // namespace
}  // namespace mednext

using namespace mednext;

extern "C" int32_t mednext_up_join_fwd(const void* main_in, const void* small, const void* bias, void* out, int64_t n,
                                       int64_t c, int64_t d, int64_t h, int64_t w, int32_t lead, int32_t dtype,
                                       void* stream) {
  if (int st = check_join(n, c, d, h, w, lead, dtype)) return st;
  MEDNEXT_CHECK_ARG(main_in != nullptr && small != nullptr && out != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG((reinterpret_cast<uintptr_t>(out) & 15u) == 0, "out must be 16-byte aligned");
  hipLaunchKernelGGL(up_join_fwd_kernel, dim3(static_cast<unsigned>(n * c * d)), dim3(kThreads), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(main_in),
                     static_cast<const uint16_t*>(small), static_cast<const uint16_t*>(bias),
                     static_cast<uint16_t*>(out), make_join(c, d, h, w, lead));
  MEDNEXT_CHECK_LAUNCH();
  return MEDNEXT_STATUS_OK;
}

extern "C" size_t mednext_up_join_bwd_workspace_bytes(int64_t n, int64_t c, int64_t d) {
  if (n < 1 || c < 1 || d < 1) return 0;
  return static_cast<size_t>(n * c * d) * sizeof(float);
}

extern "C" int32_t mednext_up_join_bwd(const void* grad_out, void* grad_main, void* grad_small, void* grad_bias,
                                       void* workspace, size_t workspace_bytes, int64_t n, int64_t c, int64_t d,
                                       int64_t h, int64_t w, int32_t lead, int32_t bias_over_grid, int32_t dtype,
                                       void* stream) {
  if (int st = check_join(n, c, d, h, w, lead, dtype)) return st;
  MEDNEXT_CHECK_ARG(bias_over_grid == 0 || bias_over_grid == 1, "bias_over_grid must be 0 or 1");
  MEDNEXT_CHECK_ARG(grad_out != nullptr && grad_main != nullptr && grad_small != nullptr, "null tensor pointer");
  MEDNEXT_CHECK_ARG((reinterpret_cast<uintptr_t>(grad_out) & 15u) == 0, "grad_out must be 16-byte aligned");
  MEDNEXT_CHECK_ARG(workspace != nullptr && workspace_bytes >= mednext_up_join_bwd_workspace_bytes(n, c, d),
                    "workspace too small");
  const JoinGeom g = make_join(c, d, h, w, lead, bias_over_grid);
  const auto s = static_cast<hipStream_t>(stream);
  float* part = static_cast<float*>(workspace);
  hipLaunchKernelGGL(up_join_bwd_kernel, dim3(static_cast<unsigned>(n * c * d)), dim3(kThreads), 0, s,
                     static_cast<const uint16_t*>(grad_out), static_cast<uint16_t*>(grad_main),
                     static_cast<uint16_t*>(grad_small), part, g);
  MEDNEXT_CHECK_LAUNCH();
  if (grad_bias != nullptr) {
    hipLaunchKernelGGL(up_join_bias_kernel, dim3(static_cast<unsigned>(c)), dim3(64), 0, s, part,
                       static_cast<uint16_t*>(grad_bias), n, g);
    MEDNEXT_CHECK_LAUNCH();
  }
  return MEDNEXT_STATUS_OK;
}
