/*
 * mednext_hip.h — C ABI of libmednext_hip.so, the gfx950 (MI355X) kernels behind
 * the MedNeXt operator path.
 *
 * Conventions (shared by every entry point):
 *   - Pointers are device pointers allocated by the caller (PyTorch's caching
 *     allocator in the Python host). The library never allocates: entry points
 *     that need scratch memory expose a *_workspace_bytes() query and take a
 *     caller-owned workspace.
 *   - Tensors are contiguous NCDHW (pointwise: [N, C, V] with V = D*H*W).
 *   - `stream` is a hipStream_t (the caller's current stream); launches are
 *     asynchronous and never synchronise.
 *   - Return value is a mednext_status; on failure mednext_hip_last_error()
 *     returns a message for the calling thread.
 *   - Reductions (weight/bias/norm gradients) are deterministic: fixed-order
 *     two-pass fp32/fp64 reductions, no floating-point atomics.
 */
#ifndef MEDNEXT_HIP_H
#define MEDNEXT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum mednext_status {
  MEDNEXT_STATUS_OK = 0,
  MEDNEXT_STATUS_INVALID_ARGUMENT = 1,
  MEDNEXT_STATUS_LAUNCH_ERROR = 2,
  MEDNEXT_STATUS_UNSUPPORTED = 3
};

/* Depthwise compute engine. VALU: fp32/fp64 FMA stencil, every dtype.
 * MFMA: bf16 banded-Toeplitz matrix-core kernels (k in {3,5}, W % 8 == 0,
 * W >= 32, H >= 32, one (n, c) slab < 2 GiB; weight-grad also W % 32 == 0);
 * tile_w is then the columns per workgroup (32, 64 or 128).
 * VOLUME: small planes (H * W <= 256, e.g. the 16^3 and 8^3 MedNeXt stages),
 * every dtype: one workgroup of k waves (one per kernel row) per (n, c) slab,
 * band of 64 consecutive plane positions and D-run, its zero-padded input rows
 * staged in LDS; tile_w must be 64 (plane positions per workgroup) and
 * depth_chunk is the D-run of one workgroup (its staged planes must fit
 * 64 KiB of LDS). */
enum mednext_engine { MEDNEXT_ENGINE_VALU = 0, MEDNEXT_ENGINE_MFMA = 1, MEDNEXT_ENGINE_VOLUME = 2 };

enum mednext_dtype {
  MEDNEXT_DTYPE_F32 = 0,
  MEDNEXT_DTYPE_F64 = 1,
  MEDNEXT_DTYPE_F16 = 2,
  MEDNEXT_DTYPE_BF16 = 3
};

/* Message for the last failing call on this host thread ("" if none). */
const char* mednext_hip_last_error(void);

/* ABI revision of this header; bumped on any signature change. */
int32_t mednext_hip_abi_version(void);

/* ------------------------------------------------------------------ depthwise
 * Depthwise Conv3d, stride 1, odd cubic kernel k in {1,3,5}, zero "same"
 * padding k/2, groups == C. weight is [C,1,k,k,k] and bias [C], both in the
 * same dtype as x (the reference casts them to x.dtype before its op).
 * engine (mednext_engine), tile_w (VALU: 4, 8, 16, 32 or 64 output columns per
 * workgroup; MFMA: 32, 64 or 128) and depth_chunk (output planes per
 * workgroup, >= 1) are the launch recipe chosen by the gfx950 tile policy.
 */

/* y = conv3d(x, weight, bias, padding=k//2, groups=C).
 * Replaces the forward of mednext_accel::depthwise_conv3d_odd_regular
 * (reference src/mednext_accel/ops/_triton/depthwise.py:549-563, which calls
 * F.conv3d). bias may be NULL. */
int32_t mednext_depthwise3d_fwd(const void* x, const void* weight, const void* bias, void* y,
                                int64_t n, int64_t c, int64_t d, int64_t h, int64_t w,
                                int32_t kernel_size, int32_t dtype, int32_t engine,
                                int32_t tile_w, int32_t depth_chunk, void* stream);

/* grad_input = conv3d(grad_output, flip(weight), padding=k//2, groups=C).
 * Replaces mednext_accel::depthwise_input_grad_odd_regular
 * (reference ops/_triton/depthwise.py:159-203 kernel, :486-513 op). */
int32_t mednext_depthwise3d_dgrad(const void* grad_output, const void* weight, void* grad_input,
                                  int64_t n, int64_t c, int64_t d, int64_t h, int64_t w,
                                  int32_t kernel_size, int32_t dtype, int32_t engine,
                                  int32_t tile_w, int32_t depth_chunk, void* stream);

/* grad_input = the input gradient above + accumulate (a bf16 tensor shaped
 * like grad_input), in one pass: MFMA engine, bf16, k in {3, 5}. The
 * MedNeXt block's input receives the depthwise input gradient and the
 * gradient of its residual; the reference's autograd adds the two
 * (models/blocks.py:82-91 uses x twice), here the add rides on the
 * depthwise kernel's store. */
int32_t mednext_depthwise3d_dgrad_acc(const void* grad_output, const void* weight, const void* accumulate,
                                      void* grad_input, int64_t n, int64_t c, int64_t d, int64_t h, int64_t w,
                                      int32_t kernel_size, int32_t dtype, int32_t engine, int32_t tile_w,
                                      int32_t depth_chunk, void* stream);

/* Bytes of fp32 (fp64 for MEDNEXT_DTYPE_F64) partials the wgrad launch needs
 * (0 if the shape / recipe is unsupported). The MFMA engine additionally needs
 * W % 32 == 0. */
size_t mednext_depthwise3d_wgrad_workspace_bytes(int64_t n, int64_t c, int64_t d, int64_t h,
                                                 int64_t w, int32_t kernel_size, int32_t dtype,
                                                 int32_t engine, int32_t tile_w,
                                                 int32_t depth_chunk);

/* grad_weight[c,t] = sum x[n,c,pos+t-p] * grad_output[n,c,pos] (dtype of x) and,
 * when grad_bias != NULL, grad_bias[c] = sum grad_output[n,c,:] — fused in the
 * same pass. Replaces mednext_accel::depthwise_weight_grad_odd_regular
 * (reference ops/_triton/depthwise.py:13-83 kernels, :445-483 op) plus the
 * native bias gradient the reference requests from aten.convolution_backward
 * (:612-633). */
int32_t mednext_depthwise3d_wgrad(const void* x, const void* grad_output, void* grad_weight,
                                  void* grad_bias, void* workspace, size_t workspace_bytes,
                                  int64_t n, int64_t c, int64_t d, int64_t h, int64_t w,
                                  int32_t kernel_size, int32_t dtype, int32_t engine,
                                  int32_t tile_w, int32_t depth_chunk, void* stream);

/* Allocation-free variant of mednext_depthwise3d_wgrad (same kernels, same
 * results bit for bit). No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). The fp32 / fp64 partials
 * live in a library-owned device array of
 * mednext_depthwise3d_wgrad_noalloc_max_bytes() bytes (16 MiB) per GPU, held
 * from the first call on that GPU until the process ends; shapes whose
 * partials need more (see mednext_depthwise3d_wgrad_workspace_bytes) are
 * rejected with MEDNEXT_STATUS_INVALID_ARGUMENT. The call allocates nothing.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (other streams, other host threads) race and must be serialised by the
 * caller. `stream` must belong to the current device. */
size_t mednext_depthwise3d_wgrad_noalloc_max_bytes(void);

int32_t mednext_depthwise3d_wgrad_noalloc(const void* x, const void* grad_output, void* grad_weight,
                                          void* grad_bias, int64_t n, int64_t c, int64_t d, int64_t h,
                                          int64_t w, int32_t kernel_size, int32_t dtype, int32_t engine,
                                          int32_t tile_w, int32_t depth_chunk, void* stream);

/* ---------------------------------------------------------------- group norm
 * GroupNorm with groups == channels on [N, C, V] (V = spatial volume), biased
 * variance, rstd = 1/sqrt(var + eps). Replaces the reference's
 * nn.GroupNorm(in_channels, in_channels) inside MedNeXtBlock (reference
 * src/mednext_accel/models/blocks.py:74, :84), which has no custom op in the
 * reference. x and y dtypes are independent so a bf16 input can produce the
 * fp32 output autocast gives the reference (pairs: f64/f64, f32/f32, bf16/f32,
 * bf16/bf16, f16/f32, f16/f16). gamma/beta (nullable) are [C] in param_dtype.
 * mean/rstd are [N*C] fp32 (fp64 when x is fp64). `splits` chunks each (n, c)
 * row across workgroups (1..4096).
 */
size_t mednext_group_norm_workspace_bytes(int64_t n, int64_t c, int64_t spatial, int32_t splits);

int32_t mednext_group_norm_fwd(const void* x, int32_t x_dtype, const void* gamma, const void* beta,
                               int32_t param_dtype, void* y, int32_t y_dtype, void* mean,
                               void* rstd, int64_t n, int64_t c, int64_t spatial, double eps,
                               int32_t splits, void* workspace, size_t workspace_bytes,
                               void* stream);

/* The forward's statistics without its output: mean / rstd as
 * mednext_group_norm_fwd writes them (bit-identical), and coef [N*C][4] fp64
 * (8-byte aligned) = (rstd * gamma, beta, mean, rstd), so GroupNorm(x) =
 * (x - mean) * (rstd * gamma) + beta per (n, c): the records of the pointwise
 * NORM prologue, which folds the normalisation into the expand GEMM and
 * reproduces mednext_group_norm_fwd's bf16 output bit for bit (reference
 * models/blocks.py:74, :84-86 norm -> conv1). Same workspace as the
 * forward. */
int32_t mednext_group_norm_stats(const void* x, int32_t x_dtype, const void* gamma, const void* beta,
                                 int32_t param_dtype, void* mean, void* rstd, void* coef, int64_t n,
                                 int64_t c, int64_t spatial, double eps, int32_t splits, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* grad_input (dtype of x, nullable), grad_gamma / grad_beta ([C], param_dtype,
 * nullable) from grad_output (pairs dy/x: f64/f64, f32/f32, f32/bf16, bf16/bf16,
 * f32/f16, f16/f16) and the saved mean/rstd. */
int32_t mednext_group_norm_bwd(const void* grad_output, int32_t dy_dtype, const void* x,
                               int32_t x_dtype, const void* mean, const void* rstd,
                               const void* gamma, int32_t param_dtype, void* grad_input,
                               void* grad_gamma, void* grad_beta, int64_t n, int64_t c,
                               int64_t spatial, int32_t splits, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------- depthwise s2
 * Stride-2, padding k/2 depthwise maps between a full-resolution tensor `big`
 * [N][C][Db][Hb][Wb] and a half-resolution tensor `small` [N][C][Ds][Hs][Ws]
 * (any sizes; out-of-range taps read zero), k in {1,3,5}, weight [C,1,k,k,k]
 * and bias [C] in the tensors' dtype, fp32 accumulation (fp64 for fp64):
 *   gather:  small[o] = bias + sum_t w[t] big[2o + t - k/2]
 *   scatter: big[i]   = bias + sum_{o,t: 2o + t - k/2 = i} w[t] small[o]
 *   wgrad:   grad_weight[t] = sum_{n,o} big[2o + t - k/2] small[o],
 *            grad_bias = sum_{n,o} small[o]
 * The MedNeXt down block's Conv3d(stride 2) is gather (forward), scatter
 * (input gradient, bias NULL) and wgrad(big = x, small = grad_output); the up
 * block's ConvTranspose3d(stride 2), whose output is 2s - 1 per dimension, is
 * scatter (forward), gather (input gradient) and wgrad(big = grad_output,
 * small = x) for the weight (its bias gradient is the sum of grad_output).
 * Kernels: bf16 maps with big = 2 small (down block) or 2 small - 1 (up
 * block) per dimension, Hb, Wb >= 32, an even Wb a multiple of 32 or an odd
 * Wb with Ws % 8 == 0, and a small plane above 256 positions (128^3 / 64^3
 * stages) run the matrix-core stride-1 kernels (gather: stencil over big,
 * even outputs stored; scatter: flipped-tap stencil over small expanded with
 * zeros; wgrad: weight gradient with dy = small expanded with zeros); small
 * planes of up to 256 positions the band kernels; the rest row-task kernels.
 * The workspace query follows the same choice.
 * Replace the reference's F.conv3d / F.conv_transpose3d forwards and their
 * backward kernels (src/mednext_accel/ops/_triton/depthwise.py:206-268,
 * :516-546, :654-719 stride-2; :86-156, :722-850 transposed). */
int32_t mednext_depthwise3d_s2_gather(const void* big, const void* weight, const void* bias,
                                      void* small_out, int64_t n, int64_t c, int64_t db,
                                      int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                      int32_t kernel_size, int32_t dtype, void* stream);
int32_t mednext_depthwise3d_s2_scatter(const void* small, const void* weight, const void* bias,
                                       void* big_out, int64_t n, int64_t c, int64_t db,
                                       int64_t hb, int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                       int32_t kernel_size, int32_t dtype, void* stream);
size_t mednext_depthwise3d_s2_wgrad_workspace_bytes(int64_t n, int64_t c, int64_t db, int64_t hb,
                                                    int64_t wb, int64_t ds, int64_t hs, int64_t ws,
                                                    int32_t kernel_size, int32_t dtype);
int32_t mednext_depthwise3d_s2_wgrad(const void* big, const void* small, void* grad_weight,
                                     void* grad_bias, void* workspace, size_t workspace_bytes,
                                     int64_t n, int64_t c, int64_t db, int64_t hb, int64_t wb,
                                     int64_t ds, int64_t hs, int64_t ws, int32_t kernel_size,
                                     int32_t dtype, void* stream);

/* ------------------------------------------------------------------ pointwise
 * 1x1x1 convolution as a per-sample GEMM on bf16 matrix cores (fp32
 * accumulate): x [N][K][V], y [N][M][V] (V = D*H*W voxels), weight [M][K]
 * (weight_layout 0) or [K][M] (weight_layout 1, i.e. the transposed product
 * for the input gradient: grad_x = W^T . grad_y with W the conv's [M][K]).
 * Requirements: bf16, 1 <= K <= 2048, any M >= 1 and V >= 1 (a row's last
 * partial 8-voxel group uses element accesses), one sample's x and y each
 * < 2 GiB, bf16-aligned tensors and a 16-byte aligned weight. K up to 8192
 * runs the tiled product (see mednext_pw_kernels) and needs what it needs:
 * K % 32 == 0, M % 16 == 0, no GELU / AFFINE / NORM prologue, no
 * ROW_REDUCE, blocks_per_sample 0 and the AUTO or TILED choice.
 * Prologue, applied to every x element as loaded:
 *   MEDNEXT_PW_PROLOGUE_GELU: x -> GELU(x) (exact erf form).
 *   MEDNEXT_PW_PROLOGUE_AFFINE: x -> bf16(fma(x, s, t)), (s, t) = entries 0
 *     and 1 of the fp64 record prologue_coef[(n * K + k) * 4] taken as
 *     floats (the records mednext_grn_stats writes: a GRN folded into the
 *     GEMM that consumes it).
 *   MEDNEXT_PW_PROLOGUE_NORM: x -> bf16(fma(x - c, s, t)), (s, t, c) =
 *     entries 0, 1 and 2 as floats (the records mednext_group_norm_stats
 *     writes: a GroupNorm(C, C) folded into the GEMM that consumes it).
 *   Both give the value the unfolded normalisation stores, bit for bit.
 *   Forward epilogues with AFFINE / NORM: BIAS, BIAS_GELU, BIAS_RESIDUAL,
 *   BIAS_GELU_PAIR, with a [M][K] weight (weight_layout 0) and K <= 2048.
 * Epilogue, applied to each accumulator y[n][m][v] (bias may be NULL):
 *   BIAS:          y = acc + bias[m]
 *   BIAS_GELU:     y = GELU(acc + bias[m])
 *   BIAS_RESIDUAL: y = acc + bias[m] + aux[n][m][v]
 *   GELU_GRAD:     y = acc * GELU'(aux[n][m][v])   (bias unused)
 *   ROW_REDUCE:    y is not written; per row, row_partial receives the fp64
 *                  pair (sum_v acc * aux, sum_v acc), one pair per slot:
 *                  row_partial[((n * M + m) * slots + slot) * 2]
 *                  (slots from mednext_pointwise_row_slots; bias unused)
 *   AFFINE_SCALE:  y = (acc * c0 + aux * c1) * aux2[n][m][v] with
 *                  (c0, c1) = epilogue_coef[(n * M + m) * 2 + {0, 1}] (fp64;
 *                  bias unused)
 *   BIAS_GELU_PAIR: y = GELU(acc + bias[m]) and y2 = GELU'(acc + bias[m])
 *   AUX_SCALE:     y = acc * aux[n][m][v]   (bias unused; with aux = GELU'(h)
 *                  stored by BIAS_GELU_PAIR, the input gradient through GELU)
 */
enum mednext_pw_prologue {
  MEDNEXT_PW_PROLOGUE_NONE = 0,
  MEDNEXT_PW_PROLOGUE_GELU = 1,
  MEDNEXT_PW_PROLOGUE_AFFINE = 2,
  MEDNEXT_PW_PROLOGUE_NORM = 3
};
enum mednext_pw_epilogue {
  MEDNEXT_PW_EPILOGUE_BIAS = 0,
  MEDNEXT_PW_EPILOGUE_BIAS_GELU = 1,
  MEDNEXT_PW_EPILOGUE_BIAS_RESIDUAL = 2,
  MEDNEXT_PW_EPILOGUE_GELU_GRAD = 3,
  MEDNEXT_PW_EPILOGUE_ROW_REDUCE = 4,
  MEDNEXT_PW_EPILOGUE_AFFINE_SCALE = 5,
  MEDNEXT_PW_EPILOGUE_BIAS_GELU_PAIR = 6,
  MEDNEXT_PW_EPILOGUE_AUX_SCALE = 7
};

/* y = epilogue(op(W) . prologue(x)); blocks_per_sample = workgroups along V
 * per (sample, output row group), 0 = the library's choice (two resident
 * workgroups per CU over the whole grid).
 * Replaces the forward of AdaptivePointwise3d (reference
 * src/mednext_accel/ops/adaptive.py:174-200: per-sample addmm / F.conv3d) and,
 * with the epilogues, the GELU (models/blocks.py:39-41) and residual add
 * (blocks.py:89-90) around it; with weight_layout 1 it is the conv's input
 * gradient (the backward of the same addmm). */
int32_t mednext_pointwise_fwd(const void* x, const void* weight, const void* bias, const void* aux,
                              void* y, int64_t n, int64_t k, int64_t m, int64_t v,
                              int32_t weight_layout, int32_t prologue, int32_t epilogue,
                              int32_t dtype, int32_t blocks_per_sample, void* stream);

/* mednext_pointwise_fwd with the extra operands of the AFFINE prologue and
 * the ROW_REDUCE / AFFINE_SCALE / BIAS_GELU_PAIR epilogues (NULL where the
 * chosen mode does not use them). Together they run the MedNeXt v2 block
 * expansion project(GRN(GELU(expand(x)))) (reference models/blocks_v2.py:44-45
 * with ops/grn.py:16-30 between the GEMMs) without a GRN output tensor: the
 * expand GEMM writes GELU and GELU' of its output, the project GEMM applies the
 * GRN affine as it loads, and in the backward one transposed GEMM reduces the
 * GRN row sums and a second writes the gradient through GRN and GELU
 * (reference ops/_triton/grn.py:242-317 plus the GELU backward). */
int32_t mednext_pointwise_fwd_ex(const void* x, const void* weight, const void* bias, const void* aux,
                                 const void* aux2, void* y, void* y2, int64_t n, int64_t k, int64_t m,
                                 int64_t v, int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                 const void* prologue_coef, const void* epilogue_coef,
                                 void* row_partial, int32_t dtype, int32_t blocks_per_sample,
                                 void* stream);

/* mednext_pointwise_fwd_ex with a caller workspace (16-byte aligned) for the
 * tiled product's K split: where the tiled grid alone would leave the chip
 * short of 256 workgroups, K is split over workgroups that write fp32 tile
 * partials to the workspace, and a second kernel adds them in a fixed order
 * and applies the epilogue. With a NULL or too small workspace it behaves as
 * mednext_pointwise_fwd_ex. No counterpart in the reference (its GEMMs are
 * library calls). */
int32_t mednext_pointwise_fwd_ws(const void* x, const void* weight, const void* bias, const void* aux,
                                 const void* aux2, void* y, void* y2, int64_t n, int64_t k, int64_t m,
                                 int64_t v, int32_t weight_layout, int32_t prologue, int32_t epilogue,
                                 const void* prologue_coef, const void* epilogue_coef,
                                 void* row_partial, int32_t dtype, int32_t blocks_per_sample,
                                 void* workspace, size_t workspace_bytes, void* stream);
/* Workspace bytes mednext_pointwise_fwd_ws uses for this shape and mode under
 * the current kernel choice (0: no K split). */
size_t mednext_pointwise_fwd_workspace_bytes(int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                             int32_t epilogue);

/* Kernel family for mednext_pointwise_fwd(_ex). The streaming kernels keep X
 * out of LDS and read it once per group of 16-64 output rows; the tiled
 * kernel stages X and the weight through LDS for 64 or 128 output rows at a
 * time (K % 32 == 0, M % 16 == 0, no GELU prologue, no ROW_REDUCE, and
 * blocks_per_sample == 0). AUTO takes the tiled kernel for K >= 256 where
 * the streaming plan would read X twice or more and the tiled grid has at
 * least 256 workgroups, and (given the workspace of mednext_pointwise_fwd_ws)
 * for K >= 256 with a smaller grid, K split over workgroups; TILED takes it
 * wherever it applies; STREAMING never. The tiled
 * kernel applies the AFFINE / NORM prologue to X as it stages it. The
 * same choice governs the weight gradient's tile: AUTO uses 128 x 128
 * workgroup tiles when M >= 128, K >= 128 and the grid keeps at least 256
 * workgroups, TILED whenever both sides exceed 32,
 * STREAMING never (64 x 64 at most). No counterpart in the reference (its
 * GEMMs are library calls); process-wide, for measurement and tests. */
enum mednext_pw_kernels {
  MEDNEXT_PW_KERNELS_AUTO = 0,
  MEDNEXT_PW_KERNELS_STREAMING = 1,
  MEDNEXT_PW_KERNELS_TILED = 2,
  MEDNEXT_PW_KERNELS_TILED_64 = 3 /* TILED with 64-row workgroups; 64 x 64 weight-gradient tiles */
};
int32_t mednext_pointwise_set_kernels(int32_t choice);
/* 1 if a launch of this shape and mode (blocks_per_sample 0) runs the tiled
 * kernel under the current choice, else 0. */
int32_t mednext_pointwise_uses_tiled(int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                     int32_t epilogue);

/* Slots per (sample, row) the ROW_REDUCE epilogue writes for this launch
 * shape (0 on invalid arguments). */
int64_t mednext_pointwise_row_slots(int64_t n, int64_t k, int64_t m, int64_t v,
                                    int32_t blocks_per_sample);

/* Bytes of workspace the weight-gradient launch needs: its fp32 per-split
 * partials, which one reduction launch sums in fixed order (fp64) into the
 * bf16 gradients. */
size_t mednext_pointwise_wgrad_workspace_bytes(int64_t n, int64_t k, int64_t m, int64_t v,
                                               int32_t splits);

/* grad_weight[M][K] = sum_{n,v} grad_output[n][m][v] * prologue(x[n][k][v]);
 * grad_bias[m] = sum_{n,v} grad_output[n][m][v] (skipped when NULL). Both bf16;
 * fixed-order reduction (bit-reproducible). splits = workgroups per sample
 * along V. Any K, M >= 1; the workspace must be 8-byte aligned. Replaces the weight/bias gradient of the reference's pointwise
 * conv (adaptive.py:174-200, autograd of addmm / conv3d). */
int32_t mednext_pointwise_wgrad(const void* grad_output, const void* x, void* grad_weight,
                                void* grad_bias, void* workspace, size_t workspace_bytes,
                                int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                int32_t dtype, int32_t splits, void* stream);

/* mednext_pointwise_wgrad with the prologue's coefficient records (AFFINE:
 * the GRN output computed from its input as the x operand; NORM: the
 * GroupNorm output). For AFFINE / NORM the product runs on the raw x and the
 * fixed-order reduction maps each per-sample sum exactly:
 * sum_v dy x' = s * sum_v dy x + (t - c s) * sum_v dy, in fp64 with the
 * records' float values (no bf16 rounding of x'). */
int32_t mednext_pointwise_wgrad_ex(const void* grad_output, const void* x, void* grad_weight,
                                   void* grad_bias, void* workspace, size_t workspace_bytes,
                                   int64_t n, int64_t k, int64_t m, int64_t v, int32_t prologue,
                                   const void* prologue_coef, int32_t dtype, int32_t splits,
                                   void* stream);

/* ------------------------------------------------------------------ GRN
 * Global Response Normalization of MedNeXt v2 on [N, C, V]:
 *   n_c = ||x[n, c, :]||_2, S = sum_c n_c, r_c = n_c / (S + eps),
 *   y = x + gamma_c * x * r_c + beta_c
 * computed in fp32 from f16/bf16/f32 input (fp64 for fp64), y in x's dtype.
 * Replaces the reference's fused Triton GRN (reference
 * src/mednext_accel/ops/_triton/grn.py:177-229 forward, :242-317 backward)
 * behind the formula of ops/grn.py:16-30. gamma/beta ([C], param_dtype,
 * nullable = 0) are the (1, C, 1, 1, 1) parameters read flat. `coef` receives
 * [N*C][4] fp64 (1 + gamma r, beta, r, n_c) for the backward. `splits` chunks
 * each (n, c) row across workgroups (1..4096); workspace is 8-byte aligned. */
size_t mednext_grn_workspace_bytes(int64_t n, int64_t c, int64_t spatial, int32_t splits);

int32_t mednext_grn_fwd(const void* x, int32_t x_dtype, const void* gamma, const void* beta,
                        int32_t param_dtype, void* y, void* coef, int64_t n, int64_t c,
                        int64_t spatial, double eps, int32_t splits, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Statistics only (no output tensor): coef as mednext_grn_fwd writes it, for
 * a consumer that applies the GRN itself (the AFFINE pointwise prologue).
 * Same workspace as mednext_grn_fwd. */
int32_t mednext_grn_stats(const void* x, int32_t x_dtype, const void* gamma,
                          const void* beta, int32_t param_dtype, void* coef, int64_t n, int64_t c,
                          int64_t spatial, double eps, int32_t splits, void* workspace,
                          size_t workspace_bytes, void* stream);

/* The GRN backward's per-(n, c) coefficients from row sums a GEMM epilogue
 * produced (row_partial [N][C][slots][2] fp64 = partial (sum dy * y_in,
 * sum dy), see MEDNEXT_PW_EPILOGUE_ROW_REDUCE): coef_out [N][C][2] fp64 =
 * (1 + gamma r, (gamma g / (S + eps) - T / (S + eps)^2) / n_c), and the
 * parameter gradients grad_gamma / grad_beta ([C], param_dtype, nullable).
 * workspace: N * C * 4 doubles. */
int32_t mednext_grn_bwd_rows(const void* row_partial, int64_t slots, const void* coef,
                             const void* gamma, int32_t param_dtype, void* coef_out,
                             void* grad_gamma, void* grad_beta, int64_t n, int64_t c, double eps,
                             void* workspace, size_t workspace_bytes, void* stream);

/* grad_input (x's dtype, nullable), grad_gamma / grad_beta ([C], param_dtype,
 * nullable) from grad_output (pairs dy/x: same dtype, or f32 with bf16/f16 x),
 * x and the forward's coef, including the cross-channel term through S and a
 * zero subgradient where n_c == 0. Fixed-order reductions (bit-reproducible). */
int32_t mednext_grn_bwd(const void* grad_output, int32_t dy_dtype, const void* x, int32_t x_dtype,
                        const void* coef, const void* gamma, int32_t param_dtype,
                        void* grad_input, void* grad_gamma, void* grad_beta, int64_t n, int64_t c,
                        int64_t spatial, double eps, int32_t splits, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------ up-block join
 * The tail of a MedNeXt up block, bf16: out [N][C][D][H][W] (D, H even, W a
 * multiple of 8) = pad(main) + pad(residual), where main is the block's
 * [N][C][D-1][H-1][W-1] output, the residual is the stride-2 transposed
 * 1x1x1 conv with bias b [C] (nullable) whose GEMM output y = W^T x + b at
 * the even grid points is small [N][C][D/2][H/2][W/2], and the pad is one
 * voxel per dimension at the start (lead 1, MedNeXt v1) or at the end (lead
 * 0, v2). Replaces the F.pad / conv_transpose3d / add sequence of the
 * reference's up blocks (models/blocks.py:176-181, models/blocks_v2.py:128-133).
 * The backward writes grad_main (on the grid), grad_small (the even grid
 * points) and, when grad_bias != NULL, grad_bias = the sum of grad_out over
 * the other grid points, or with bias_over_grid = 1 over the whole
 * (D-1)(H-1)(W-1) grid (fixed-order fp64 reduction of per-plane fp32
 * partials in the caller's workspace, rounded once). bias_over_grid is for a
 * caller that computed small with the bias's value but routes the bias's
 * gradient here: the sum is then its whole gradient, one rounding, as the
 * reference's conv_transpose3d bias reduction. */
int32_t mednext_up_join_fwd(const void* main_in, const void* small, const void* bias, void* out, int64_t n,
                            int64_t c, int64_t d, int64_t h, int64_t w, int32_t lead, int32_t dtype,
                            void* stream);
size_t mednext_up_join_bwd_workspace_bytes(int64_t n, int64_t c, int64_t d);
int32_t mednext_up_join_bwd(const void* grad_out, void* grad_main, void* grad_small, void* grad_bias,
                            void* workspace, size_t workspace_bytes, int64_t n, int64_t c, int64_t d,
                            int64_t h, int64_t w, int32_t lead, int32_t bias_over_grid, int32_t dtype,
                            void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MEDNEXT_HIP_H */
