// Internal interface between the depthwise C-ABI entry points and the bf16
// matrix-core kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mednext {

// True when the MFMA kernels handle this volume and kernel size.
bool dw_mfma_supported(int64_t d, int64_t h, int64_t w, int k);

// bf16 depthwise stencil on MFMA: forward (flip = false, bias nullable) or
// input gradient (flip = true, bias = nullptr). tile_cols in {32, 64, 128}.
// With acc != nullptr (input gradient): y = stencil + acc.
int dw_mfma_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n,
                    int64_t c, int64_t d, int64_t h, int64_t w, int k, bool flip, int tile_cols,
                    int depth_chunk, hipStream_t st, const void* acc = nullptr);

// Number of per-workgroup partials per channel the MFMA wgrad writes (0 if the
// shape or recipe is unsupported).
int dw_mfma_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k,
                         int tile_cols, int depth_chunk);

// bf16 weight gradient (+ bias-grad sums) on MFMA into fp32 partials laid out
// [C][k^3 + 1][splits]; reduce with the shared finish kernel.
int dw_mfma_wgrad(const void* x, const void* dy, float* partial, int64_t n, int64_t c, int64_t d,
                  int64_t h, int64_t w, int k, int tile_cols, int depth_chunk, hipStream_t st);

// Stride-2 maps (the down block's depthwise conv) on the same kernels, bf16:
// gather small[o] = b + sum_t w[t] big[2o + t - p], scatter big[i] = b +
// sum_{2o + t - p = i} w[t] small[o], and the weight gradient dW[t] = sum_o
// big[2o + t - p] small[o] (+ dB = sum small) into [C][k^3 + 1][splits] fp32
// partials. Supported: k in {3, 5}, big = 2 * small or 2 * small - 1 per
// dimension (down block / up block), H, W >= 32, even big W a multiple of 32,
// odd big W with a small W multiple of 8, slabs < 2 GiB.
bool dw_mfma_s2_supported(int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k);
int dw_mfma_s2_gather(const void* big, const void* weight, const void* bias, void* small, int64_t n, int64_t c,
                      int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st);
int dw_mfma_s2_scatter(const void* small, const void* weight, const void* bias, void* big, int64_t n, int64_t c,
                       int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st);
int dw_mfma_s2_wgrad_splits(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                            int64_t ws, int k);
int dw_mfma_s2_wgrad(const void* big, const void* small, float* partial, int64_t n, int64_t c, int64_t db, int64_t hb,
                     int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, hipStream_t st);

}  // namespace mednext
