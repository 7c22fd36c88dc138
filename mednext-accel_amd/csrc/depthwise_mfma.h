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

}  // namespace mednext
