// Internal interface between the depthwise C-ABI entry points and the
// small-plane kernels (depthwise_volume.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mednext {

// True when the volume kernels take this plane (H * W <= 256 elements).
bool dw_volume_supported(int64_t h, int64_t w);

// Forward (flip = false, bias nullable) or input gradient (flip = true, bias =
// nullptr) of one depthwise layer, any dtype. seg must be 4 (output planes per
// lane); depth_chunk is the D-run of one workgroup.
int dw_volume_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n, int64_t c, int64_t d,
                      int64_t h, int64_t w, int k, int dtype, bool flip, int seg, int depth_chunk, hipStream_t st);

// Partials per channel the volume weight gradient writes (0 if unsupported).
int dw_volume_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int seg,
                           int depth_chunk);

// Weight gradient and bias-gradient sums into accumulation-type partials laid
// out [C][k^3 + 1][splits]; reduce with the shared finish kernel.
int dw_volume_wgrad(const void* x, const void* dy, void* partial, int64_t n, int64_t c, int64_t d, int64_t h,
                    int64_t w, int k, int dtype, int seg, int depth_chunk, hipStream_t st);

}  // namespace mednext
