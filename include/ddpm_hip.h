/*
 * ddpm_hip.h - C ABI of libddpm_hip.so, the MI355X (gfx950) DDPM hot path.
 *
 * Every entry point takes plain device pointers, int64 sizes and a HIP
 * stream; none allocates, none synchronizes; launches are asynchronous on
 * `stream`.  Each returns 0 on success, a hipError_t value on a launch
 * failure, or one of the DDPM_STATUS_* codes below (ddpm_status_string()
 * turns any code into text).  Tensors are contiguous:
 *
 *   x, y, grad_x, grad_y        [N][C][H][W]
 *   kernels, grad_kernels       [N][3][C][K*K][H][W]   (row o = (b*C+c)*K*K + ki*K + kj)
 *   weight, grad_weight         [3*C*K*K][C]           (Conv2d [3CK^2, C, 1, 1])
 *   bias, grad_bias             [3*C*K*K]
 *   out / grad_out ("cat")      [N][4*C][H][W] = [x, d0, d1, d2]
 *
 * dtype codes: 0 = float32, 1 = bfloat16, 2 = float16; 3 = float32 whose
 * concat ("cat") is stored as bf16 pair planes -- per 32-plane chunk, plane
 * j < 16 holds the hi halves of channels (2j, 2j+1) (low / high 16 bits) and
 * plane 16 + j their lo halves, hi = the top 16 bits of the fp32 pattern and
 * lo = the remainder rounded to nearest even (the split the fp32 MFMA path
 * makes of its operands).  Code 3 is taken where noted: by ddpm_gen_fwd
 * (writes such a concat; c % 16 == 0), ddpm_fuse_conv_fwd and
 * ddpm_fuse_conv_bwd_weight (read one; c % 8 == 0) and their workspace
 * queries (as code 0); the other tensors of those calls are float32.
 * Dilations d0, d1, d2 are the three branch dilations ((1, 3, 5) in DDPM).
 * The neighbour of (h, w) for tap (ki, kj) at dilation d is
 * (h + (ki - K/2) d, w + (kj - K/2) d), zero outside the image.
 */
#ifndef DDPM_HIP_H
#define DDPM_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DDPM_STATUS_OK 0
#define DDPM_STATUS_BAD_ARGUMENT 10001
#define DDPM_STATUS_UNSUPPORTED 10002
#define DDPM_STATUS_WORKSPACE_TOO_SMALL 10003
#define DDPM_STATUS_SCRATCH_TOO_SMALL 10004

#define DDPM_DTYPE_F32 0
#define DDPM_DTYPE_BF16 1
#define DDPM_DTYPE_F16 2

/* ABI version of this header (5: dtype code 3; 6: ddpm_gen_fwd at K = 5 and
 * ddpm_gen_fwd_supported; 7: ddpm_fuse_conv_bwd, ddpm_gen_fwd_pack and
 * ddpm_fuse_conv_fwd_packed). */
int ddpm_abi_version(void);

/* Text for any status code returned by this library (static storage). */
const char* ddpm_status_string(int code);

/* 1 when the fused generator entry points (ddpm_gen_*) accept this channel
 * count, kernel size and largest dilation (C <= 128, K in {1, 3}, and for
 * K = 3 max_dilation <= 8, the column halo the backward kernels stage; a 1x1
 * tap ignores the dilation), else 0.  The reference's fused path has no
 * channel limit; callers route other shapes to the materialized entry points
 * (ddpm_filter_*), with identical results. */
int ddpm_gen_supported(int64_t c, int kernel_size, int max_dilation);

/* 1 when ddpm_gen_fwd alone -- the fused forward, for inference -- accepts
 * this channel count, kernel size and largest dilation (C <= 128, K in {1, 3,
 * 5}, the halo tile of radius (K/2)*max_dilation within one workgroup's LDS:
 * max_dilation <= 12 at K = 3, <= 6 at K = 5), else 0; host-only.  The
 * reference's module fuses inference at any K (triton_impl.py:317-338, the
 * fused forward _triton_kernels.py:268-300); training above K = 3
 * materializes the kernels there as here. */
int ddpm_gen_fwd_supported(int64_t c, int kernel_size, int max_dilation);

/* 1 when ddpm_gen_kernels and ddpm_gen_kernels_bwd_w accept this shape and
 * dtype (c <= 128, one image's generated planes within 2^31 - 1 bytes, grids
 * below 2^31 workgroups), else 0; host-only.  Callers compute other shapes
 * with a library convolution.  Part of the routing of the reference's
 * materialized path (triton_impl.py:340-347). */
int ddpm_gen_kernels_supported(int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                               int dtype);

/* The generator's 1x1 convolution on the materialized route:
 * kernels[n][o][p] = sum_i weight[o][i] * y[n][i][p] + bias[o] for
 * o < 3*c*k*k, rounded once to `dtype`, written in the [n][3][c][k*k][h][w]
 * layout the ddpm_filter_* entry points read.  weight: [3*c*k*k][c] (the
 * Conv2d weight without its trailing 1x1), bias: [3*c*k*k].  c <= 128
 * (kUnsupported beyond); any kernel size.
 * Replaces the cuDNN 1x1 convolution self.generator(y) of the reference's
 * materialized path (triton_impl.py:340-347). */
int ddpm_gen_kernels(const void* y, const void* weight, const void* bias, void* kernels, int64_t n,
                     int64_t c, int64_t h, int64_t w, int kernel_size, int dtype, hipStream_t stream);

/* Weight and bias gradients of that convolution:
 * grad_weight[o][i] = sum_{n,p} grad_kernels[n][o][p] * y[n][i][p] and
 * grad_bias[o] = sum_{n,p} grad_kernels[n][o][p], accumulated in fp32 and
 * rounded once to `dtype` (deterministic: fixed-order split partials).
 * grad_kernels: [n][3*c*k*k][h][w]; grad_weight: [3*c*k*k][c]; an empty
 * batch writes zeros.  c <= 128.  Replaces the backward-filter convolution
 * of self.generator on the reference's materialized path
 * (triton_impl.py:340-347, autograd of nn.Conv2d). */
int64_t ddpm_gen_kernels_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                               int kernel_size);
int ddpm_gen_kernels_bwd_w(const void* y, const void* grad_kernels, void* grad_weight,
                           void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t n,
                           int64_t c, int64_t h, int64_t w, int kernel_size, int dtype,
                           hipStream_t stream);

/* Input gradient of that convolution: grad_y[n][i][p] =
 * sum_o weight[o][i] * grad_kernels[n][o][p], accumulated in fp32 and rounded
 * once to `dtype` (deterministic: o-split partials summed in split order).
 * weight: [3*c*k*k][c]; grad_kernels: [n][3*c*k*k][h][w] (rows whose
 * 16-byte chunks are aligned are copied to LDS directly, others element by
 * element); kUnsupported when c > 128.  Replaces the
 * backward-data convolution of self.generator on the reference's
 * materialized path (triton_impl.py:340-347, autograd of nn.Conv2d). */
int64_t ddpm_gen_kernels_bwd_y_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                               int kernel_size);
int ddpm_gen_kernels_bwd_y(const void* weight, const void* grad_kernels, void* grad_y,
                           void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                           int64_t h, int64_t w, int kernel_size, int dtype, hipStream_t stream);

/* ---- materialized dynamic filter ------------------------------------- */

/* out = [x, d0, d1, d2] from materialized kernels; out has k_dtype, and the
 * filter accumulates in fp32.
 * Replaces _dynamic_cat_fwd + _DynamicCat.forward (_triton_kernels.py:21-101, 814-842). */
int ddpm_filter_fwd(const void* x, const void* kernels, void* out, int64_t n, int64_t c, int64_t h,
                    int64_t w, int kernel_size, int d0, int d1, int d2, int x_dtype, int k_dtype,
                    hipStream_t stream);

/* grad_x[c,q] = grad_out[x-channel c, q]
 *             + sum_b sum_tap kernels[b,c,tap,q-off] * grad_out[branch b, c, q-off].
 * grad_out and kernels have k_dtype, grad_x has x_dtype.
 * Replaces _dynamic_cat_bwd_x (_triton_kernels.py:104-190, launched at :862-863). */
int ddpm_filter_bwd_x(const void* grad_out, const void* kernels, void* grad_x, int64_t n, int64_t c,
                      int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int x_dtype,
                      int k_dtype, hipStream_t stream);

/* grad_kernels[b,c,tap,p] = grad_out[branch b, c, p] * x[c, p+off(b,tap)].
 * Replaces _dynamic_cat_bwd_k (_triton_kernels.py:193-254, launched at :864-865). */
int ddpm_filter_bwd_k(const void* x, const void* grad_out, void* grad_kernels, int64_t n, int64_t c,
                      int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int x_dtype,
                      int k_dtype, hipStream_t stream);

/* ---- fused generator (all tensors share `dtype`) ---------------------- */

/* out = [x, d0, d1, d2] with the dynamic taps generated on chip
 * (gen = weight . y + bias, rounded to `dtype` for bf16/f16); dtype 3 writes
 * fp32 results as pair planes (c % 16 == 0, else kUnsupported).  K in
 * {1, 3, 5} (shapes of ddpm_gen_fwd_supported; the backward entry points take
 * K <= 3).
 * Replaces _generator_dynamic_cat_fwd + _launch_generator_dynamic_cat
 * (_triton_kernels.py:268-420, 873-908). */
int ddpm_gen_fwd(const void* x, const void* y, const void* weight, const void* bias, void* out,
                 int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                 int d2, int dtype, hipStream_t stream);

/* Bytes of workspace ddpm_gen_bwd_x needs: the fp32 partial sums of its
 * tiles, halo of radius (kernel_size/2)*max(d) included (about 1.9x the
 * fp32 size of x at dilations (1,3,5)); valid for every dtype, 0 for an
 * unsupported or empty shape.
 * Part of the launch set-up of _GeneratorDynamicCat.backward (_triton_kernels.py:944-961). */
int64_t ddpm_gen_bwd_x_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                                       int d0, int d1, int d2);

/* grad_x of the fused op, recomputing the generator once per pixel and
 * scattering its products to the shifted pixels (deterministic order).
 * `workspace` (at least ddpm_gen_bwd_x_workspace_bytes) is overwritten.
 * Replaces _generator_dynamic_cat_bwd_x (_triton_kernels.py:430-531, launched at :944-961). */
int ddpm_gen_bwd_x(const void* y, const void* weight, const void* bias, const void* grad_out,
                   void* grad_x, void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                   int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
                   hipStream_t stream);

/* Bytes of workspace ddpm_gen_bwd_y needs for its packed copy of the weight
 * (bf16 hi/lo split, MFMA fragment order); valid for every dtype.
 * Part of the launch set-up of _GeneratorDynamicCat.backward (_triton_kernels.py:963-971). */
int64_t ddpm_gen_bwd_y_workspace_bytes(int64_t c, int kernel_size);

/* grad_y = weight^T . dK with dK = grad_out[branch] * shifted x formed on chip.
 * `workspace` (at least ddpm_gen_bwd_y_workspace_bytes) receives the packed
 * weight; the call overwrites it.
 * Replaces _generator_dynamic_cat_bwd_y (_triton_kernels.py:534-623, launched at :963-971). */
int ddpm_gen_bwd_y(const void* x, const void* weight, const void* grad_out, void* grad_y,
                   void* workspace, int64_t workspace_bytes, int64_t n, int64_t c, int64_t h,
                   int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
                   hipStream_t stream);

/* ddpm_gen_bwd_y without a workspace argument: allocates nothing.
 * No counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  The packed weight goes to a fixed
 * device buffer of ddpm_gen_bwd_y_noalloc_scratch_bytes() bytes (2 MiB,
 * enough for every shape the fused kernels accept) that the library holds on
 * each device it runs on until the process ends; a shape that needs more
 * returns DDPM_STATUS_SCRATCH_TOO_SMALL.  Every call on one device shares
 * that buffer, so calls that overlap on one device (different streams, or
 * other host threads) race; calls in one stream's order do not.  Same
 * arguments otherwise, and bit-identical results to ddpm_gen_bwd_y. */
int ddpm_gen_bwd_y_noalloc(const void* x, const void* weight, const void* grad_out, void* grad_y,
                           int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, int d0,
                           int d1, int d2, int dtype, hipStream_t stream);
int64_t ddpm_gen_bwd_y_noalloc_scratch_bytes(void);

/* Bytes of workspace ddpm_gen_bwd_w needs for `dtype`: its fp32 split
 * partials (none when one split writes grad_weight / grad_bias directly; the
 * same for every dtype); 0 for an invalid dtype.
 * Replaces the partial-buffer sizing of _GeneratorDynamicCat.backward (_triton_kernels.py:1001-1017). */
int64_t ddpm_gen_bwd_w_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size,
                                       int dtype);

/* grad_weight[o,i] = sum_p dK[o,p] y[i,p], grad_bias[o] = sum_p dK[o,p]; split
 * over at most 16 token ranges (of at least 4 row segments of 128 columns)
 * into fp32 partials in `workspace`, then summed in split order
 * (deterministic); one split writes the gradients directly.
 * DDPM_STATUS_UNSUPPORTED for a dilation above 8 or 3*K*K*C*(C+1) >= 2^31.
 * Replaces _generator_dynamic_cat_bwd_weight_partial + _bwd_weight_reduce
 * (_triton_kernels.py:626-811, launched at :973-1053). */
int ddpm_gen_bwd_w(const void* x, const void* y, const void* grad_out, void* grad_weight,
                   void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                   int64_t h, int64_t w, int kernel_size, int d0, int d1, int d2, int dtype,
                   hipStream_t stream);

/* ddpm_gen_bwd_x and ddpm_gen_bwd_w in one call, with the same results bit
 * for bit: the input gradient's tile kernel runs first, and its halo
 * reduction then runs on the CUs the weight gradient's workgroups leave free
 * (at most 16 splits x 3 branches x the 16-channel blocks: 192 of 256 CUs at
 * C = 64), as extra workgroups of the weight-gradient launch, instead of as a
 * kernel of its own (a separate kernel where fewer than a quarter of the CUs
 * are free).  workspace_x / workspace_w as for the two calls; both are
 * validated before anything is launched.
 * Replaces the _generator_dynamic_cat_bwd_x launch and the weight-gradient
 * launches of _GeneratorDynamicCat.backward (_triton_kernels.py:944-961,
 * 973-1053) when both gradients are needed. */
int ddpm_gen_bwd_xw(const void* x, const void* y, const void* weight, const void* bias,
                    const void* grad_out, void* grad_x, void* grad_weight, void* grad_bias,
                    void* workspace_x, int64_t workspace_x_bytes, void* workspace_w,
                    int64_t workspace_w_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                    int kernel_size, int d0, int d1, int d2, int dtype, hipStream_t stream);

/* All four gradients of the fused op in one call (ddpm_gen_bwd_x, _bwd_y and
 * _bwd_w), bit-identical to the three calls: the dX tile kernel, then the
 * weight-gradient launch whose helper workgroups (on the CUs its own grid
 * leaves free) pack the dY kernel's weight and run dX's halo reduction, the
 * split reduction, and the dY kernel.  The three workspaces as for the
 * separate calls (workspace_y: ddpm_gen_bwd_y_workspace_bytes); all parts are
 * validated before anything is launched.
 * Replaces the three kernel launches of _GeneratorDynamicCat.backward
 * (_triton_kernels.py:944-1053). */
int ddpm_gen_bwd(const void* x, const void* y, const void* weight, const void* bias,
                 const void* grad_out, void* grad_x, void* grad_y, void* grad_weight,
                 void* grad_bias, void* workspace_x, int64_t workspace_x_bytes, void* workspace_y,
                 int64_t workspace_y_bytes, void* workspace_w, int64_t workspace_w_bytes,
                 int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                 int d2, int dtype, hipStream_t stream);

/* ---- the 3x3 fuse convolution (Conv2d(4C -> C, 3, padding 1)) -------- */

/* Bytes of workspace ddpm_fuse_conv_fwd / _bwd_data need at this shape: the
 * packed weight (MFMA fragment order; fp32 as bf16 hi / lo) and, where the
 * image is too small to fill the GPU with whole input-plane loops (e.g.
 * 128x128 C=64 forward), the fp32 partial sums of the input-plane splits,
 * summed by a second kernel in split order.  The larger of the two
 * directions, so one buffer serves both. */
int64_t ddpm_fuse_conv_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w, int dtype);

/* out[n][co][h][w] = bias[co] + sum_{ci,ki,kj} weight[co][ci][ki][kj] *
 *                    cat[n][ci][h+ki-1][w+kj-1]  (zero padding), accumulated in
 * fp32 (fp32 operands as three bf16 MFMA products) and rounded once to
 * `dtype`.  cat: [n][4c][h][w]; weight: [c][4c][3][3]; bias: [c] or NULL.
 * dtype 3: cat in pair planes (c % 8 == 0), fp32 weight, bias and out.
 * Replaces the cuDNN forward of self.fuse (triton_impl.py:294, 392). */
int ddpm_fuse_conv_fwd(const void* cat, const void* weight, const void* bias, void* out,
                       void* workspace, int64_t workspace_bytes, int64_t n, int64_t c, int64_t h,
                       int64_t w, int dtype, hipStream_t stream);

/* ddpm_gen_fwd writing the concat `out`, whose workgroups also pack the fuse
 * convolution's weight (fuse_weight: [c][4c][3][3] in the concat's element
 * type) into the start of fuse_workspace (ddpm_fuse_conv_workspace_bytes for
 * `dtype`) in the layout ddpm_fuse_conv_fwd reads over `out`; then
 * ddpm_fuse_conv_fwd_packed on the same concat and workspace is
 * ddpm_fuse_conv_fwd, bit for bit, without its packing launch.  Both parts
 * are validated before anything is launched.  No reference counterpart of
 * its own: the generator launch of _launch_generator_dynamic_cat
 * (_triton_kernels.py:873-908) followed by the forward of self.fuse
 * (triton_impl.py:392), with one launch fewer. */
int ddpm_gen_fwd_pack(const void* x, const void* y, const void* weight, const void* bias, void* out,
                      const void* fuse_weight, void* fuse_workspace, int64_t fuse_workspace_bytes,
                      int64_t n, int64_t c, int64_t h, int64_t w, int kernel_size, int d0, int d1,
                      int d2, int dtype, hipStream_t stream);

/* ddpm_fuse_conv_fwd whose workspace already holds the packed weight that
 * ddpm_gen_fwd_pack wrote for this concat (same shape, dtype and buffer). */
int ddpm_fuse_conv_fwd_packed(const void* cat, const void* bias, void* out, void* workspace,
                              int64_t workspace_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                              int dtype, hipStream_t stream);

/* grad_cat[n][ci][h][w] = sum_{co,ki,kj} weight[co][ci][ki][kj] *
 *                         grad_out[n][co][h-ki+1][w-kj+1]  (zero outside the image).
 * Replaces the cuDNN backward-data convolution of self.fuse (autograd of
 * nn.Conv2d, triton_impl.py:294, 392). */
int ddpm_fuse_conv_bwd_data(const void* grad_out, const void* weight, void* grad_cat,
                            void* workspace, int64_t workspace_bytes, int64_t n, int64_t c,
                            int64_t h, int64_t w, int dtype, hipStream_t stream);

/* Bytes of workspace ddpm_fuse_conv_bwd_weight needs for `dtype`: fp32
 * split partials of the weight and bias gradients (none with one split; the
 * same for every dtype). */
int64_t ddpm_fuse_conv_bwd_weight_workspace_bytes(int64_t n, int64_t c, int64_t h, int64_t w,
                                                  int dtype);

/* grad_weight[co][ci][ki][kj] = sum_{n,h,w} grad_out[n][co][h][w] *
 *                               cat[n][ci][h+ki-1][w+kj-1]  (zero padding),
 * grad_bias[co] = sum grad_out[n][co][h][w]; fp32 accumulation in at most 16
 * pixel splits summed in split order (deterministic), rounded once to
 * `dtype`; an empty batch writes zeros.  c <= 128 (kUnsupported beyond; above
 * 64 output planes workgroups take halves of 64).  dtype 3: cat in pair
 * planes (c % 8 == 0), bit-identical to code 0 on the same values.
 * Replaces the cuDNN backward-filter convolution of self.fuse (autograd of
 * nn.Conv2d, triton_impl.py:294, 392). */
int ddpm_fuse_conv_bwd_weight(const void* cat, const void* grad_out, void* grad_weight,
                              void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t n,
                              int64_t c, int64_t h, int64_t w, int dtype, hipStream_t stream);

/* Input, weight and bias gradients of the fuse convolution in one call
 * (ddpm_fuse_conv_bwd_weight, then ddpm_fuse_conv_bwd_data), bit-identical to
 * the two calls in two launches instead of four: the weight-gradient launch's
 * workgroups also pack the input gradient's weight, and the input-gradient
 * launch's workgroups also sum the weight gradient's split partials.
 * `dtype` is the concat's code (3: pair planes; grad_out, weight and grad_cat
 * are then plain fp32).  workspace_data as for ddpm_fuse_conv_bwd_data
 * (ddpm_fuse_conv_workspace_bytes), workspace_weight as for
 * ddpm_fuse_conv_bwd_weight; both live at once.  Both parts are validated
 * before anything is launched.
 * Replaces the cuDNN backward-data and backward-filter convolutions of
 * self.fuse (autograd of nn.Conv2d, triton_impl.py:294, 392) when all
 * gradients are needed. */
int ddpm_fuse_conv_bwd(const void* cat, const void* weight, const void* grad_out, void* grad_cat,
                       void* grad_weight, void* grad_bias, void* workspace_data,
                       int64_t workspace_data_bytes, void* workspace_weight,
                       int64_t workspace_weight_bytes, int64_t n, int64_t c, int64_t h, int64_t w,
                       int dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DDPM_HIP_H */
