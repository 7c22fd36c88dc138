// Internal interface between the depthwise C-ABI entry points and the band
// kernels (depthwise_volume.hip): small-plane stride-1 depthwise and the
// stride-2 gather / reduce maps.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mednext {

// True when the volume kernels take this plane (H * W <= 256 elements).
bool dw_volume_supported(int64_t h, int64_t w);

// Forward (flip = false, bias nullable) or input gradient (flip = true, bias =
// nullptr) of one depthwise layer, any dtype. band must be 64 (plane positions
// per workgroup); depth_chunk is the D-run of one workgroup.
int dw_volume_stencil(const void* x, const void* weight, const void* bias, void* y, int64_t n, int64_t c, int64_t d,
                      int64_t h, int64_t w, int k, int dtype, bool flip, int band, int depth_chunk, hipStream_t st);

// Partials per channel the volume weight gradient writes (0 if unsupported).
int dw_volume_wgrad_splits(int64_t n, int64_t c, int64_t d, int64_t h, int64_t w, int k, int dtype, int band,
                           int depth_chunk);

// Weight gradient and bias-gradient sums into accumulation-type partials laid
// out [C][k^3 + 1][splits]; reduce with the shared finish kernel.
int dw_volume_wgrad(const void* x, const void* dy, void* partial, int64_t n, int64_t c, int64_t d, int64_t h,
                    int64_t w, int k, int dtype, int band, int depth_chunk, hipStream_t st);

// True when the stride-2 band kernels take this big / small pair (small width
// at most ceil(big width / 2), slabs under 2 GiB, staged rows within 64 KiB).
bool dw_s2band_supported(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                         int64_t ws, int k, int dtype);

// True when the entry points should use the band kernels for this pair
// (supported and measured faster than the row-task kernels).
bool dw_s2band_chosen(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                      int64_t ws, int k, int dtype);

// small[o] = b + sum_t w[t] big[2o + t - P] (bias nullable), any dtype.
int dw_s2band_gather(const void* big, const void* weight, const void* bias, void* small, int64_t n, int64_t c,
                     int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, int dtype,
                     hipStream_t st);

// Partials per channel dw_s2band_wgrad writes (0 if unsupported).
int dw_s2band_wgrad_splits(int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb, int64_t ds, int64_t hs,
                           int64_t ws, int k, int dtype);

// dW[t] = sum_o big[2o + t - P] small[o] and dB = sum_o small[o] into
// accumulation-type partials [C][k^3 + 1][splits]; reduce with the shared
// finish kernel.
int dw_s2band_wgrad(const void* big, const void* small, void* partial, int64_t n, int64_t c, int64_t db, int64_t hb,
                    int64_t wb, int64_t ds, int64_t hs, int64_t ws, int k, int dtype, hipStream_t st);

}  // namespace mednext
