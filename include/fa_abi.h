/*
 * frame_analytics_amd -- C ABI of the MI355X (gfx950) metric kernels.
 *
 * This is the drop-in boundary for the GPU half of NevermindNilas/frame_analytics.
 * Every entry point below replaces one `fa_cuda_*` entry point of the reference's
 * C ABI (reference: frame_analytics/csrc/fa_abi.h) with the same argument list,
 * the same argument meaning and the same status codes.  Only the prefix differs:
 * `fa_gpu_` instead of `fa_cuda_`, because the library behind it is hand-written
 * HIP for CDNA4 and links nothing from CUDA.
 *
 * Conventions (identical to the reference, fa_abi.h:12-21):
 *   - every entry point returns an int status; FA_OK (0) is success
 *   - a negative status is a HIP runtime error, negated (see fa_gpu_error_string)
 *   - the caller owns every buffer, scratch included.  Python allocates them
 *     through torch's caching allocator, which keeps calls legal inside a HIP
 *     graph capture
 *   - shapes travel as ints, dtypes as an int code, streams as an opaque
 *     hipStream_t handle; the device ordinal is explicit on every call
 *   - nothing here allocates device memory and nothing synchronises
 */
#ifndef FRAME_ANALYTICS_AMD_ABI_H
#define FRAME_ANALYTICS_AMD_ABI_H

#include <stdint.h>

#define FA_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* Bumped whenever a signature below changes meaning (reference fa_abi.h:41). */
#define FA_ABI_VERSION 1

/* dtype codes (reference fa_abi.h:44-48) */
#define FA_U8 0
#define FA_F16 1
#define FA_BF16 2
#define FA_F32 3
#define FA_F64 4
/* No counterpart in the reference: a flag fa_gpu_ssim_cs_ex accepts OR-ed
 * into FA_F32 or FA_F16.  It promises that every sample is a level of the
 * 2x2-mean pyramid of uint8 data: with FA_F32 a multiple of 4^-s in [0, 255],
 * s <= 4; with FA_F16 the first level (s = 1, multiples of 1/4, exact in
 * float16).  That lets the call run on the matrix cores; without it the input
 * runs the vector-ALU kernel.  Results agree either way to the same 1e-6 bar. */
#define FA_DTYPE_U8_PYRAMID 0x100

/* pixel-loss selector (reference fa_abi.h:51-54) */
#define FA_OP_MSE 0
#define FA_OP_L1 1
#define FA_OP_CHARB 2 /* param = eps^2 */
#define FA_OP_HUBER 3 /* param = delta */

/* status codes (reference fa_abi.h:57-64); negative = -(hipError_t) */
#define FA_OK 0
#define FA_E_DTYPE 1
#define FA_E_SHAPE 2
#define FA_E_WINDOW 3
#define FA_E_OP 4
#define FA_E_ARG 5
#define FA_E_INTERNAL 6
#define FA_E_NOGPU 7
/* No counterpart in the reference: fa_gpu_ssim_noalloc's fixed scratch is too
 * small for the call (N * C * slots per plane > FA_NOALLOC_SLOTS). */
#define FA_E_SCRATCH 8

/* "not an MSE reduction, skip the dB conversion" (reference fa_abi.h:67) */
#define FA_PSNR_NONE (-1.0e300)

/* Largest supported Gaussian window; odd widths 3..11 (reference fa_abi.h:71). */
#define FA_MAX_WIN 11

/* Replaces fa_cuda_abi_version (reference fa_abi.h:131). */
FA_API int fa_gpu_abi_version(void);

/* Replaces fa_cuda_error_string (reference fa_abi.h:132). */
FA_API const char* fa_gpu_error_string(int code);

/* Replaces fa_cuda_device_count (reference fa_abi.h:133). */
FA_API int fa_gpu_device_count(int* out_count);

/*
 * Replaces fa_cuda_pixel_workspace (reference fa_abi.h:135-136).
 * out_bpi: partial slots per image of fa_gpu_pixel_reduce; `partial` must hold
 * n_images * bpi 8-byte slots.  Images of at least 4 Mi elements get one slot
 * per wave of a one-workgroup-per-CU sweep (8 x CUs); smaller ones one per
 * workgroup of a per-image grid.  Any bpi >= 1 is accepted by the reductions.
 */
FA_API int fa_gpu_pixel_workspace(int64_t n_images, int64_t n_per_image,
                                  int device, int* out_bpi);

/*
 * Replaces fa_cuda_pixel_reduce (reference fa_abi.h:140-147).
 * partial: [n_images, bpi] 8-byte scratch (uint64 bit patterns for the exact
 * uint8 MSE/L1 sums, float64 otherwise).  Any of the four sinks may be null;
 * the psnr sinks are written only when psnr_bias != FA_PSNR_NONE.
 */
FA_API int fa_gpu_pixel_reduce(const void* a, const void* b, int dtype,
                               int64_t n_images, int64_t n_per_image, int op,
                               double param, double psnr_bias, double* partial,
                               int bpi, double* out_per_image,
                               double* out_total, double* out_psnr_per_image,
                               double* out_psnr_total, int device,
                               void* stream);

/*
 * Replaces fa_cuda_ssim_workspace (reference fa_abi.h:149).
 * out_bpp: partial slots per plane of fa_gpu_ssim / fa_gpu_ssim_cs.
 */
FA_API int fa_gpu_ssim_workspace(int H, int W, int K, int* out_bpp);

/*
 * Replaces fa_cuda_ssim (reference fa_abi.h:152-159).
 * partial: [N*C, bpp] float64.  map_out: optional [N, C, H-K+1, W-K+1] float32.
 * out_per_image: N float64 (may be null).  out_total: 1 float64 (may be null).
 */
FA_API int fa_gpu_ssim(const void* x, const void* y, int dtype, int N, int C,
                       int H, int W, const float* win, int K, double shift,
                       double C1, double C2, float* map_out, double* partial,
                       int bpp, double* out_per_image, double* out_total,
                       int device, void* stream);

/*
 * Replaces fa_cuda_ssim_cs (reference fa_abi.h:162-168).
 * out_s / out_cs: N*C float64 each, per-plane means of the SSIM map and of its
 * contrast-structure factor.
 */
FA_API int fa_gpu_ssim_cs(const void* x, const void* y, int dtype, int N,
                          int C, int H, int W, const float* win, int K,
                          double shift, double C1, double C2, double* partial,
                          double* partial_cs, int bpp, double* out_s,
                          double* out_cs, int device, void* stream);

/*
 * Replaces fa_cuda_ssim_backward (reference fa_abi.h:174-181).
 * aux: (dy ? 4 : 3) * N*C * (H-K+1) * (W-K+1) float32 scratch.  Exactly one of
 * dL_dmap (full map gradient) and grad_scalar (1-element device tensor, the
 * gradient of the batch-mean SSIM) must be non-null.
 */
FA_API int fa_gpu_ssim_backward(const float* x, const float* y,
                                const float* dL_dmap, const float* grad_scalar,
                                const float* win, int K, int N, int C, int H,
                                int W, double shift, double C1, double C2,
                                float* aux, float* dx, float* dy, int device,
                                void* stream);

/*
 * Replaces fa_cuda_ssim_cs_backward (reference fa_abi.h:184-190).
 * gs / gcs: N*C float32 device scalars, dL/d(plane-mean SSIM) and
 * dL/d(plane-mean cs).
 */
FA_API int fa_gpu_ssim_cs_backward(const float* x, const float* y,
                                   const float* gs, const float* gcs,
                                   const float* win, int K, int N, int C,
                                   int H, int W, double shift, double C1,
                                   double C2, float* aux, float* dx,
                                   float* dy, int device, void* stream);

/*
 * Replaces fa_cuda_gmsd_workspace (reference fa_abi.h:192).
 * out_bpp: partial slots per plane of fa_gpu_gmsd.
 */
FA_API int fa_gpu_gmsd_workspace(int H, int W, int downsample, int* out_bpp);

/*
 * Replaces fa_cuda_gmsd (reference fa_abi.h:195-200).
 * psum / psumsq: [N*C, bpp] float64.  out_mean / out_std: N float64 each.
 */
FA_API int fa_gpu_gmsd(const void* x, const void* y, int dtype, int N, int C,
                       int H, int W, double Tc, double eps, int downsample,
                       double* psum, double* psumsq, int bpp, double* out_mean,
                       double* out_std, int device, void* stream);

/* ------------------------------------------------------------------------ */
/* Extensions: no counterpart in the reference's C ABI.                     */
/* ------------------------------------------------------------------------ */

/*
 * No counterpart in the reference, which materialises a float32 luma plane
 * (functional.py:267-271) and copies crops contiguous (backend.py:346,482).
 * fa_gpu_pixel_reduce over strided N x C x H x W views, optionally of luma:
 *   a_strides / b_strides: {image, channel, row} strides in elements (columns
 *     are contiguous), or null for contiguous;
 *   luma: {kr, kg, kb, offset} or null.  With luma, C must be 3 and each
 *     image is one plane; the term is formed from the luma difference
 *     kr dR + kg dG + kb dB in float64 (the offset cancels and is not read).
 * The mean is over (luma ? 1 : C) * H * W elements per image.  partial:
 * [n_images, bpi] with bpi from fa_gpu_pixel_workspace(n_images, C * H * W);
 * it holds uint64 exact sums for uint8 MSE / L1 without luma.
 */
FA_API int fa_gpu_pixel_reduce_ex(const void* a, const void* b, int dtype,
                                  int64_t n_images, int C, int H, int W,
                                  const int64_t* a_strides,
                                  const int64_t* b_strides, const double* luma,
                                  int op, double param, double psnr_bias,
                                  double* partial, int bpi,
                                  double* out_per_image, double* out_total,
                                  double* out_psnr_per_image,
                                  double* out_psnr_total, int device,
                                  void* stream);

/*
 * No counterpart in the reference, which materialises a float32 luma plane
 * (functional.py:267-271) and copies crops contiguous (backend.py:346,482).
 * fa_gpu_ssim over strided views, optionally of luma:
 *   x_strides / y_strides: {image, channel, row} strides in elements (columns
 *     are contiguous), or null for a contiguous N x C x H x W tensor; a plane
 *     must span fewer than 2^31 elements;
 *   luma: {kr, kg, kb, offset} or null.  With luma, C must be 3 and each
 *     image is one plane kr R + kg G + kb B + offset (offset in data units).
 * map_out / partial / outputs as fa_gpu_ssim with N * (luma ? 1 : C) planes.
 */
FA_API int fa_gpu_ssim_ex(const void* x, const void* y, int dtype, int N, int C,
                          int H, int W, const int64_t* x_strides,
                          const int64_t* y_strides, const double* luma,
                          const float* win, int K, double shift, double C1,
                          double C2, float* map_out, double* partial, int bpp,
                          double* out_per_image, double* out_total, int device,
                          void* stream);

/*
 * No counterpart in the reference, which pools its MS-SSIM pyramid with torch
 * between scales (reference functional.py:876-885).  fa_gpu_ssim_cs over
 * views with optional luma (as fa_gpu_ssim_ex), plus, when px / py are not
 * null, the next pyramid level of x and y written by the same pass:
 * non-overlapping 2x2 mean (of the luma plane, offset included, with luma),
 * odd trailing row / column dropped.  px / py:
 * N * Cout * (H/2) * (W/2) elements of pool_dtype, which is FA_F64, or FA_F32
 * for uint8 and float32 input (and for a float16 first level flagged
 * FA_DTYPE_U8_PYRAMID) without luma, or FA_F16 for uint8 input without luma
 * (the first level of a uint8 image, multiples of 1/4 in [0, 255], is exact
 * in float16).  The means are formed in float64, so the levels of a uint8
 * pyramid are exact in float32 and those of float16 / bfloat16 / float32 exact
 * in float64 (unless a 2x2 block spans more than 2^29 / 2^45 in magnitude;
 * then correctly rounded).
 * out_s / out_cs: N * Cout plane means as in fa_gpu_ssim_cs, or both null:
 * then no finalize runs and the partial sums stay in partial / partial_cs for
 * fa_gpu_ms_ssim_reduce; partial may then be null too, and the pass forms
 * the cs sums alone (MS-SSIM reads no SSIM sums below its coarsest scale).  out_slots: host int, may be null unless both means
 * are null; receives the number of slots per plane the launch used (each
 * plane's partial sums are packed at that stride from the start of the
 * buffer).  dtype: FA_F32 | FA_DTYPE_U8_PYRAMID marks a uint8 pyramid level,
 * FA_F16 | FA_DTYPE_U8_PYRAMID its first level in float16 (see
 * FA_DTYPE_U8_PYRAMID).
 */
FA_API int fa_gpu_ssim_cs_ex(const void* x, const void* y, int dtype, int N,
                             int C, int H, int W, const int64_t* x_strides,
                             const int64_t* y_strides, const double* luma,
                             const float* win, int K, double shift, double C1,
                             double C2, double* partial, double* partial_cs,
                             int bpp, double* out_s, double* out_cs,
                             int* out_slots, void* px, void* py,
                             int pool_dtype, int device, void* stream);

/*
 * No counterpart in the reference, which materialises a float32 luma plane
 * before GMSD (functional.py:267-271) and copies crops contiguous
 * (backend.py:346,482).  fa_gpu_gmsd over strided views, optionally of luma:
 *   x_strides / y_strides: {image, channel, row} strides in elements (columns
 *     are contiguous), or null for a contiguous N x C x H x W tensor;
 *   luma: {kr, kg, kb, offset} or null.  With luma, C must be 3 and each
 *     image is one plane kr R + kg G + kb B, formed in float64 (the offset
 *     cancels out of every gradient and is not read).
 * map_out: null, or the similarity map q, float32 [N * (luma ? 1 : C), Hout,
 * Wout] with Hout x Wout the 'valid' Prewitt grid of the (downsampled) image.
 * psum / psumsq: [N * (luma ? 1 : C), bpp] float64 with bpp from
 * fa_gpu_gmsd_workspace; out_mean / out_std: N float64 each.
 */
FA_API int fa_gpu_gmsd_ex(const void* x, const void* y, int dtype, int N, int C,
                          int H, int W, const int64_t* x_strides,
                          const int64_t* y_strides, const double* luma,
                          double Tc, double eps, int downsample, float* map_out,
                          double* psum, double* psumsq, int bpp,
                          double* out_mean, double* out_std, int device,
                          void* stream);

/*
 * No counterpart in the reference.  fa_gpu_ssim_cs_backward for x / y / dx / dy
 * of element type `dtype` (FA_F32 or FA_F64, the exact pyramid levels), plus
 * the gradient of the level fa_gpu_ssim_cs_ex derived from them: gpx / gpy
 * (either may be null), (H/2) x (W/2) per plane of gp_dtype (FA_F32 or
 * FA_F64), each value spread as 1/4 over its 2x2 block of dx / dy.  aux stays
 * float32 with the same size as in fa_gpu_ssim_cs_backward.
 */
FA_API int fa_gpu_ssim_cs_backward_ex(const void* x, const void* y, int dtype,
                                      const float* gs, const float* gcs,
                                      const float* win, int K, int N, int C,
                                      int H, int W, double shift, double C1,
                                      double C2, const void* gpx,
                                      const void* gpy, int gp_dtype,
                                      float* aux, void* dx, void* dy,
                                      int device, void* stream);

/*
 * No counterpart in the reference, whose MS-SSIM training path runs the CS
 * forward of every scale and, in the backward, a coefficient pass before the
 * scatter (fa_cuda.cu:655-784 per scale).  MS-SSIM's loss reads one plane mean
 * per scale (cs below the coarsest scale, SSIM there), and the coefficient
 * maps are linear in that mean's gradient.  This pass is the CS forward of
 * fa_gpu_ssim_cs_ex in float64 (x / y of `dtype` FA_F32 or FA_F64, contiguous
 * N x C x H x W, no luma) -- plane means out_s / out_cs (N * C float64) from
 * `partial` / `partial_cs` (bpp slots per plane, fa_gpu_ssim_workspace), and
 * optionally the next pyramid level px / py of `pool_dtype` (FA_F32 or
 * FA_F64) -- which also writes into `aux` the coefficient maps of
 * fa_gpu_ssim_cs_backward for a unit gradient of the SSIM means (unit_s != 0)
 * or of the cs means (unit_s == 0): b, c, tx and, with aux_dy, ty, each
 * N * C * Hout * Wout float32.
 */
FA_API int fa_gpu_ssim_cs_coef(const void* x, const void* y, int dtype, int N,
                               int C, int H, int W, const float* win, int K,
                               double shift, double C1, double C2, int unit_s,
                               double* partial, double* partial_cs, int bpp,
                               double* out_s, double* out_cs, void* px,
                               void* py, int pool_dtype, float* aux,
                               int aux_dy, int device, void* stream);

/*
 * No counterpart in the reference (see fa_gpu_ssim_cs_coef).  The scatter of
 * fa_gpu_ssim_cs_backward over the maps fa_gpu_ssim_cs_coef wrote, each
 * plane's share times gscale[plane] (N * C float64: the upstream gradient of
 * that plane's mean), plus the pyramid level's gradient gpx / gpy as in
 * fa_gpu_ssim_cs_backward_ex.  dy needs maps written with aux_dy.
 */
FA_API int fa_gpu_ssim_cs_scatter(const void* x, const void* y, int dtype,
                                  const double* gscale, const float* win, int K,
                                  int N, int C, int H, int W, double shift,
                                  const float* aux, int aux_dy, const void* gpx,
                                  const void* gpy, int gp_dtype, void* dx,
                                  void* dy, int device, void* stream);

/*
 * No counterpart in the reference, whose GMS / GMSD losses differentiate the
 * portable PyTorch path (modules.py:183-184).  Gradients of
 *   L = sum_n g_mean[n] * mean_n(q) + g_std[n] * std_n(q)
 * with respect to contiguous x and y (N x C x H x W of dtype FA_F32 or
 * FA_F64), computed in float64.  mean / std_dev: fa_gpu_gmsd's outputs for
 * the same inputs (device, N each); g_mean / g_std: device arrays of N (either
 * may be null: zero); aux: 4 * N*C*Hout*Wout float64 scratch; dx / dy: either
 * may be null, written in full (zero on the row / column a downsample drops).
 */
FA_API int fa_gpu_gmsd_backward(const void* x, const void* y, int dtype, int N,
                                int C, int H, int W, double Tc, double eps,
                                int downsample, const double* mean,
                                const double* std_dev, const double* g_mean,
                                const double* g_std, double* aux, void* dx,
                                void* dy, int device, void* stream);

/*
 * No counterpart in the reference, which reduces every MS-SSIM scale in a
 * finalize launch of its own and combines the scales with torch ops
 * (functional.py:897-901).  From the partial sums fa_gpu_ssim_cs_ex left
 * (out_s = out_cs = null): per plane t_j = (sum of its slots) / npix[j],
 * prod_j max(t_j, 0)^w_j, the mean over the C channels of each image and the
 * batch mean of those, in two launches.
 *   partials: host array of M (<= 8) device pointers, scale j's partial_cs
 *     (partial, the SSIM sums, for the coarsest scale), N * C * slots[j]
 *     float64 each;
 *   slots / npix / weights: host arrays of M: slots per plane (out_slots of
 *     that scale's call), output pixels of one plane, and the weights;
 *   plane_scratch: M * N * C float64 device scratch;
 *   out_per_image (N) / out_total (1) float64: either may be null, not both.
 */
FA_API int fa_gpu_ms_ssim_reduce(const double* const* partials,
                                 const int* slots, const double* npix,
                                 const double* weights, int M, int N, int C,
                                 double* plane_scratch, double* out_per_image,
                                 double* out_total, int device, void* stream);

/*
 * No counterpart in the reference, which combines the MS-SSIM scales with
 * torch ops (functional.py:897-901).  The same head as the end of
 * fa_gpu_ms_ssim_reduce over plane means that are already formed (the
 * training path, where each scale's means come out of its own pass): per
 * plane prod_j max(t_j, 0)^w_j (a NaN mean stays NaN), the mean over the C
 * channels of each image and the batch mean of those, in one launch.
 *   terms: host array of M (<= 8) device pointers, scale j's plane means
 *     (N * C float64: cs below the coarsest scale, SSIM at it);
 *   weights: host array of M;
 *   out_per_image (N) / out_total (1) float64: either may be null, not both.
 */
FA_API int fa_gpu_ms_ssim_head(const double* const* terms, int M, int N, int C,
                               const double* weights, double* out_per_image,
                               double* out_total, int device, void* stream);

/*
 * No counterpart in the reference (see fa_gpu_ms_ssim_head).  Its gradient,
 * in one launch: from the upstream gradient of the per-image values
 * (g_per_image, N float64) or of the batch mean (g_total, 1 float64; exactly
 * one of the two), each scale's gradient of its plane means into g_terms[j]
 * (host array of M device pointers, N * C float64 each; a null entry is not
 * written).  The clamp and the power differentiate as torch's clamp_min and
 * pow: 0 where t_j < 0, t_j is NaN or w_j = 0, and inf for a zero mean under
 * a fractional weight; the product's derivative multiplies the other factors
 * (exact where some are zero).
 */
FA_API int fa_gpu_ms_ssim_head_backward(const double* const* terms, int M,
                                        int N, int C, const double* weights,
                                        const double* g_per_image,
                                        const double* g_total,
                                        double* const* g_terms, int device,
                                        void* stream);

/*
 * No counterpart in the reference, whose MS-SSIM is a Python loop over the
 * scales with torch pooling between them (functional.py:874-901).  The
 * inference MS-SSIM in one call: for each of the M (<= 8) scales the fused
 * pass of fa_gpu_ssim_cs_ex (the cs sums; the SSIM sums at the coarsest
 * scale; the next pyramid level, exact: float16 for the first level and
 * float32 below it under uint8 input, float64 under floating input or a luma
 * plane), then the reduction of fa_gpu_ms_ssim_reduce, launched back to back
 * with no host work between them.  x / y: N x C x H x W of any dtype, with
 * optional strides and luma as in fa_gpu_ssim_ex; weights: host array of M.
 * workspace: at least fa_gpu_ms_ssim_workspace's bytes of device memory
 * (levels, partial sums, scratch).  Every scale's shape is checked before
 * anything is launched.  out_per_image (N) / out_total (1) float64: either
 * may be null, not both.
 *
 * acc: null, or FA_MS_SSIM_ACC_WORDS uint64 of device memory, zero when the
 * call starts; the call leaves it zero.  With it, uint8 input without luma
 * whose every scale fits the matrix-core kernel (widths a multiple of 8 at
 * every scale, e.g. W % 128 == 0 at M = 5; K <= 16; C1, C2 > 0; N * C <= 256;
 * 3 <= M <= 5) runs as three launches: scale 0, scale 1 (which also writes
 * levels 3 and 4), and scales 2 .. M - 1 side by side in one launch whose last
 * workgroup finishes the reduction from per-(scale, plane) fixed-point sums
 * (about 1e-13 relative from the float64 reduction, the same bits run to run).
 * Other calls ignore acc.  `acc` is state of one stream: calls that overlap
 * on it (two streams, graph replays beside eager calls) race.  After a
 * non-zero status its contents are unknown (a failure between the launches
 * leaves words set): zero it again before the next call.
 */
#define FA_MS_SSIM_ACC_WORDS ((8 * 256 + 1) * 16)
FA_API int fa_gpu_ms_ssim_workspace(int dtype, int N, int C, int H, int W, int K, int M,
                                    int luma, int64_t* out_bytes);
FA_API int fa_gpu_ms_ssim(const void* x, const void* y, int dtype, int N, int C, int H, int W,
                          const int64_t* x_strides, const int64_t* y_strides,
                          const double* luma, const float* win, int K, double shift,
                          double C1, double C2, const double* weights, int M, void* workspace,
                          int64_t workspace_bytes, uint64_t* acc, double* out_per_image,
                          double* out_total, int device, void* stream);

/*
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc: fa_gpu_ssim (same arguments, same results, the same
 * kernels) without the `partial` / `bpp` workspace.  The partial sums go to
 * a fixed scratch array in the library, FA_NOALLOC_SLOTS float64 (8 MiB) per
 * GPU, held by each GPU the library runs on until the process ends; the call
 * itself allocates nothing.  A call needing more than N * C * (slots per
 * plane, fa_gpu_ssim_workspace) > FA_NOALLOC_SLOTS returns FA_E_SCRATCH
 * before touching the GPU (e.g. up to ~480 1080p planes at K = 11).
 * Calls on one GPU share its scratch: calls that overlap on one GPU (two
 * streams, two threads) race and must be serialised by the caller.  The first
 * call on a device looks up the scratch array's address there (which may
 * load the code object); made on a stream under graph capture it returns
 * FA_E_ARG and does nothing, so one eager call on the device must come before
 * a capture.  After it the entry point can be captured and replayed.
 */
#define FA_NOALLOC_SLOTS (1 << 20)
FA_API int fa_gpu_ssim_noalloc(const void* x, const void* y, int dtype, int N,
                               int C, int H, int W, const float* win, int K,
                               double shift, double C1, double C2,
                               float* map_out, double* out_per_image,
                               double* out_total, int device, void* stream);

/*
 * No counterpart in the reference, whose pixel reductions always end in a
 * separate finalize launch (fa_cuda.cu:1150-1155).  fa_gpu_pixel_reduce (same
 * arguments, same results bit for bit) plus `acc`: FA_PIXEL_ACC_WORDS uint64
 * of device memory that is zero when the call starts and that the call leaves
 * zero when it completes.  Where the sums are exact -- dtype FA_U8, op
 * FA_OP_MSE or FA_OP_L1, contiguous batches the one-workgroup-per-CU sweep
 * takes (images of >= 4 Mi elements, 16-byte aligned), at most 32 images --
 * the sweep finishes the call itself: each workgroup adds its per-image sums
 * to `acc` with returning device-scope atomics, and the workgroup that adds
 * an image's last sum writes that image's outputs (and the batch's, after the
 * batch's last image).  One launch instead of two.  Every other call ignores
 * `acc` (it may be null) and runs as fa_gpu_pixel_reduce.  `acc` is state of
 * one stream: calls that may overlap (two streams) need one buffer each.
 * `partial` may be null for a call that takes the one-launch form (it is not
 * read); a call with a null `partial` that cannot returns FA_E_ARG before
 * launching anything.
 */
#define FA_PIXEL_ACC_WORDS ((32 + 1) * 16)
FA_API int fa_gpu_pixel_reduce_once(const void* a, const void* b, int dtype,
                                    int64_t n_images, int64_t n_per_image, int op,
                                    double param, double psnr_bias, double* partial,
                                    int bpi, uint64_t* acc, double* out_per_image,
                                    double* out_total, double* out_psnr_per_image,
                                    double* out_psnr_total, int device, void* stream);

/*
 * No counterpart in the reference, whose GMSD ends in a finalize launch
 * (fa_cuda.cu:1460-1465) and whose batch means are torch ops
 * (functional.py:1082).  fa_gpu_gmsd_ex without the map (same arguments and
 * per-image results), plus
 *   acc: FA_GMSD_ACC_WORDS uint64 of device memory, zero when the call starts,
 *     left zero when it completes (state of one stream, like
 *     fa_gpu_pixel_reduce_once's);
 *   out_batch: optional double[2], the batch means of out_mean and out_std.
 * Without the map, with T or eps positive and N <= 64, the kernel finishes
 * the call itself (any input dtype; a NaN or inf sample flags its image,
 * whose statistics and the batch means then come out NaN, as the float64
 * sums would): each workgroup adds its sums of d = 1 - q and d^2 to
 * `acc` as round-to-nearest fixed-point integers (so the result does not
 * depend on the order of the adds) with returning device-scope atomics, and
 * the workgroups that complete an image's sums write its statistics (the
 * batch means likewise).  The per-image values then differ from
 * fa_gpu_gmsd's fixed-order float64 sums by the fixed-point rounding, about
 * 2^-52 relative per workgroup.  Every other call runs fa_gpu_gmsd_ex's
 * launches (plus one block for out_batch) and ignores `acc`.  psum / psumsq
 * may be null for a call that finishes in its launch; one with them null that
 * cannot returns FA_E_ARG before launching anything.
 */
#define FA_GMSD_ACC_WORDS ((3 * 64 + 2) * 16)
FA_API int fa_gpu_gmsd_once(const void* x, const void* y, int dtype, int N, int C, int H,
                            int W, const int64_t* x_strides, const int64_t* y_strides,
                            const double* luma, double Tc, double eps, int downsample,
                            double* psum, double* psumsq, int bpp, uint64_t* acc,
                            double* out_mean, double* out_std, double* out_batch, int device,
                            void* stream);

/*
 * No counterpart in the reference, whose SSIM ends in a finalize launch
 * (fa_cuda.cu:1218-1222).  fa_gpu_ssim_ex (same arguments and results), plus
 * acc: FA_SSIM_ACC_WORDS uint64 of device memory, zero when the call starts
 * and left zero when it completes (state of one stream, like
 * fa_gpu_pixel_reduce_once's).  A call with no map, N <= 256, a mean
 * wanted and C1, C2 > 0 (so that no SSIM value is NaN) finishes in its one
 * launch -- the matrix-core forward's (uint8 planes without luma, 8-sample
 * aligned rows; see fa_gpu_ssim) or the strip kernel's (every other input,
 * luma and views included, while C_out * tiles per image stays below 4096):
 * each workgroup adds its sum of the map to `acc` as a round-to-nearest
 * signed fixed-point integer (so the result does not depend on the order of
 * the adds) with returning device-scope atomics, and the workgroups that
 * complete an image's sum, and the batch's, write the means.  They differ
 * from fa_gpu_ssim's fixed-order float64 sums by that rounding, ~1e-13
 * relative at 1080p.  A workgroup sum that is not finite (NaN or inf in
 * floating input) sets a flag beside the image's word instead, and that
 * image's mean and the batch mean come out NaN, as the float64 sums would.
 * Every other call runs as fa_gpu_ssim_ex and ignores
 * `acc`.  `partial` may be null for a call that finishes in its launch; one
 * with a null `partial` that cannot returns FA_E_ARG before launching anything.
 */
#define FA_SSIM_ACC_WORDS ((256 + 1) * 16)
FA_API int fa_gpu_ssim_once(const void* x, const void* y, int dtype, int N, int C, int H,
                            int W, const int64_t* x_strides, const int64_t* y_strides,
                            const double* luma, const float* win, int K, double shift,
                            double C1, double C2, float* map_out, double* partial, int bpp,
                            uint64_t* acc, double* out_per_image, double* out_total,
                            int device, void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* FRAME_ANALYTICS_AMD_ABI_H */
