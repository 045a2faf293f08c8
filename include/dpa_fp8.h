/*
 * dpa_fp8.h — C ABI of the MI355X (gfx950) FP8 conv/GEMM path.
 *
 * Every entry point:
 *   - takes raw device pointers, explicit sizes and a hipStream_t passed as void*;
 *   - launches asynchronously on that stream and never synchronises the host;
 *   - allocates nothing: outputs and workspaces are owned by the caller;
 *   - returns DPA_OK (0), a negative DPA_E* code when a precondition fails (nothing is
 *     launched), or a positive hipError_t when a launch fails.
 *
 * Tensor conventions (all dense, no padding between rows):
 *   activations  NHWC    ([N][H][W][C], C contiguous)  — the reference's channels_last
 *   conv weights OHWI    ([Cout][R][S][Cin])          — channels_last of (Cout, Cin, R, S)
 *   e4m3         OCP float8_e4m3fn bytes (bias 7, max 448, 0x7f/0xff = NaN)
 *   bf16         IEEE bfloat16 bits, round-to-nearest-even
 *   scales       one fp32 value in device memory ("0-dim tensor")
 *
 * Reference interfaces replaced (fattorib/diffusion-profiled, diffusion/fp8_kernels.py):
 *   dpa_quantize_fp8_bf16          <- quantize_fp8                        :559-601 (K1+K2+K3)
 *   dpa_quantize_fp8_delayed_bf16  <- quantize_fp8_delayed                :518-556 (K4+K2)
 *   dpa_quantize_fp8_delayed_window_bf16, dpa_window_max3_f32
 *                                  <- the amax-window updates of diffusion/unet.py:72-91
 *                                     and fp8_kernels.py:849, :888-889 (torch ops there)
 *   dpa_conv2d_fwd_fp8             <- conv2d_fwd_fp8_prequantized         :604-639 (K5)
 *   dpa_conv2d_dgrad_fp8           <- conv2d_bwd_input_fp8_prequantized   :671-709 (K6)
 *   dpa_conv2d_wgrad_fp8           <- conv2d_bwd_weight_fp8_prequantized  :723-808 (K7+K8+K9)
 *   dpa_gemm_fp8                   <- no reference kernel; the FP8 recipe applied to the
 *                                     nn.Linear sites of diffusion/unet.py:171-172
 *   dpa_gn_silu_fwd_bf16 / _bwd    <- nn.GroupNorm + F.silu (+ FiLM) of diffusion/unet.py:151,
 *                                     :157-159 (Inductor-fused in the reference)
 *   dpa_gn_silu_fwd_fp8 / _bwd_fp8, dpa_residual_scale_bwd_fp8
 *                                  <- those producers with the delayed-scaling cast of the
 *                                     conv they feed folded in (fp8_kernels.py:856, :885-893)
 */
#ifndef DPA_FP8_H
#define DPA_FP8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DPA_OK 0
#define DPA_ERR_NULL (-1)        /* a required pointer is NULL */
#define DPA_ERR_SIZE (-2)        /* a size is negative, zero where not allowed, or too large */
#define DPA_ERR_ALIGN (-3)       /* a pointer lacks the alignment the kernel needs */
#define DPA_ERR_SHAPE (-4)       /* shape combination the kernels do not implement */
#define DPA_ERR_WORKSPACE (-5)   /* workspace missing or smaller than *_workspace_bytes() */

/* Human-readable text for a status code (static storage). */
const char* dpa_status_string(int status);

/* ABI version of this library; bumped when a signature changes. */
int dpa_abi_version(void);

/* ------------------------------------------------------------------------------------------
 * Per-tensor absmax scaling and e4m3 cast.
 *   scale = amax > 0 ? RN32(amax / 448) : 1            (fp8_kernels.py:90-102)
 *   q[i]  = e4m3_RNE( max(-448, min(RN32(f32(x[i]) / scale), 448)) )   (:105-120)
 * Bit-exact: q and scale are identical to the CPU restatement for every bf16 input.
 * x and q have the same (dense) memory order; they are treated as flat arrays of n items.
 * ---------------------------------------------------------------------------------------- */

/* Bytes of workspace the two quantize entry points need for n elements. */
int64_t dpa_quant_workspace_bytes(int64_t n);

/* Current scaling: scale_out <- scale(amax(x)); q <- cast(x, scale_out).
 * Replaces quantize_fp8 (diffusion/fp8_kernels.py:559-601). Two launches. */
int dpa_quantize_fp8_bf16(const void* x, int64_t n, void* q, float* scale_out,
                          void* workspace, int64_t workspace_bytes, void* stream);

/* Current scaling whose amax pass ran in the kernel that wrote x: partials[0..np) are that
 * kernel's per-workgroup maxima of |x| as bf16 magnitude bits (|x| & 0x7fff; the LayerNorm
 * and attention *_amax entries below leave them). One launch, the cast of
 * dpa_quantize_fp8_bf16 (quantize_fp8_kernel, diffusion/fp8_kernels.py:105-120, with the
 * finalize :90-102 over the partials): the same q and scale_out when the partials cover x.
 * 1 <= np <= 2^20. */
int dpa_quantize_fp8_bf16_from_partials(const void* x, int64_t n, const void* partials, int np,
                                        void* q, float* scale_out, void* stream);

/* Current scaling with no workspace argument and no allocation: the same launches, bytes and
 * scale as dpa_quantize_fp8_bf16, with the amax partials in a fixed 4 KB device array of the
 * library (dpa_quantize_fp8_bf16_noalloc_scratch_bytes(); one copy per GPU, held until the
 * process ends; its device address is looked up once per device on the first call there).
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, serving loops, harnesses that forbid hipMalloc). Calls no hipMalloc,
 * hipFree or allocating library routine. Every n > 0 fits: the amax pass's grid, and so the
 * partial count (dpa_quant_partials_count(n)), is at most 256, and the array holds 1024; a
 * size whose workspace would exceed the array returns DPA_ERR_WORKSPACE. All calls
 * on one GPU share the array: calls that overlap on that GPU (concurrent streams, threads)
 * race and must be serialised by the caller. The stream's device (or the current device for
 * the NULL stream) selects the array. */
int64_t dpa_quantize_fp8_bf16_noalloc_scratch_bytes(void);
int dpa_quantize_fp8_bf16_noalloc(const void* x, int64_t n, void* q, float* scale_out,
                                  void* stream);

/* Delayed scaling: q <- cast(x, *prev_scale); cur_scale_out <- scale(amax(x)).
 * One read of x. Replaces quantize_fp8_delayed (diffusion/fp8_kernels.py:518-556). */
int dpa_quantize_fp8_delayed_bf16(const void* x, int64_t n, const float* prev_scale, void* q,
                                  float* cur_scale_out, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/* dpa_quantize_fp8_delayed_bf16 plus the amax-window update of the delayed-scaling module:
 * window[*window_pos] <- cur_scale, then, if advance_pos, *window_pos <- (*window_pos + 1) %
 * window_len (window_pos is the module's int64 position tensor). Replaces the
 * scatter_ / add_ / remainder_ of diffusion/unet.py:82-91 (weights, acts) and
 * diffusion/fp8_kernels.py:888-889 (dy); the window update rides on the finalize launch. */
int dpa_quantize_fp8_delayed_window_bf16(const void* x, int64_t n, const float* prev_scale,
                                         void* q, float* cur_scale_out, float* window,
                                         int64_t* window_pos, int64_t window_len,
                                         int advance_pos, void* workspace,
                                         int64_t workspace_bytes, void* stream);

/* out3[i] <- torch.max(w_i) over n floats, for three windows in one launch (NaN if a window
 * holds one). Replaces the torch.max(amax_window_*) of diffusion/unet.py:72-73 and
 * diffusion/fp8_kernels.py:849. */
int dpa_window_max3_f32(const float* w0, const float* w1, const float* w2, int64_t n,
                        float* out3, void* stream);

/* ------------------------------------------------------------------------------------------
 * FP8 implicit-GEMM convolution, NHWC activations, OHWI weights, fp32 accumulation,
 * fused dequant epilogue:  out = bf16_RNE( RN32(acc * RN32(sa * sb)) [+ bias[c]] ).
 * Supported: R = S = 3 with pad 1 and stride 1 or 2;  R = S = 1 with pad 0, stride 1.
 * Cin and Cout must be multiples of 128 (the MFMA K depth and output tile).
 * Output size P = (H + 2*pad - R) / stride + 1, Q likewise.
 * ---------------------------------------------------------------------------------------- */

/* y[N,P,Q,Cout] = conv(xq[N,H,W,Cin], wq[Cout,R,S,Cin]).
 * Replaces conv2d_fwd_fp8_prequantized (diffusion/fp8_kernels.py:604-639) and its kernel
 * conv2d_fwd_fp8_kernel (:142-247). bias may be NULL (the reference has none). */
int dpa_conv2d_fwd_fp8(const void* xq, const void* wq, const float* x_scale,
                       const float* w_scale, const float* bias, void* y, int N, int H, int W,
                       int Cin, int Cout, int R, int S, int stride, int pad, void* stream);

/* Fragment-native e4m3 weights for the 3x3 / stride-1 / pad-1 convolutions of 16- or
 * 32-pixel-wide images (the U-Net's 32x32 and 16x16 levels): the layout the conv kernel's
 * per-wave weight loads read as contiguous 1 KB runs, so a weight's bytes are re-laid once
 * per weight update instead of being gathered per K-step. wf: the forward weight; wf_dgrad:
 * the data gradient's (transposed, taps mirrored). Same bytes as the OHWI weight, permuted:
 * 2 KB blocks, block (kc * R*S + t) * (rows / 16) + rb holds at byte h * 1024 + l * 16 + b
 * row 16 rb + (l % 16), K byte 128 kc + 32 (l / 16) + 16 h + b of tap t, where forward rows
 * are Cout and K is Cin (w[co][t][ci]) and data-gradient rows are Cin and K is Cout
 * (w[co][R*S-1-t][ci]). Either output may be NULL. Cin, Cout multiples of 128.
 * No reference counterpart: it replaces the per-call weight transpose the data gradient
 * needs (transpose_fp8_2d's role for dy, diffusion/fp8_kernels.py:321-337, applied to w). */
int64_t dpa_weight_frag_bytes(int Cout, int R, int S, int Cin);
int dpa_weight_frag_fp8(const void* wq, void* wf, void* wf_dgrad, int Cout, int R, int S,
                        int Cin, void* stream);

/* dpa_conv2d_fwd_fp8 / dpa_conv2d_dgrad_fp8 for R = S = 3, stride 1, pad 1, W in {16, 32},
 * H a multiple of 256 / W, with the weight in its fragment layout (dpa_weight_frag_fp8):
 * identical results. Other shapes return DPA_ERR_SHAPE. y / dx 16-B aligned. */
int dpa_conv2d_fwd_fp8_wf(const void* xq, const void* wf, const float* x_scale,
                          const float* w_scale, const float* bias, void* y, int N, int H,
                          int W, int Cin, int Cout, void* stream);
int dpa_conv2d_dgrad_fp8_wf(const void* dyq, const void* wf_dgrad, const float* dy_scale,
                            const float* w_scale, void* dx, int N, int H, int W, int Cin,
                            int Cout, void* stream);

/* Bytes of workspace dpa_conv2d_dgrad_fp8 needs (the transposed weight, Cout*R*S*Cin). */
int64_t dpa_conv2d_dgrad_workspace_bytes(int Cin, int Cout, int R, int S);

/* dx[N,H,W,Cin] = conv_transpose(dyq[N,P,Q,Cout], wq[Cout,R,S,Cin]); H, W are the INPUT
 * spatial sizes of the forward conv. Replaces conv2d_bwd_input_fp8_prequantized
 * (diffusion/fp8_kernels.py:671-709) and conv2d_dx_fp8_kernel (:250-318).
 * The workspace receives wq transposed to [Cin][R][S][Cout]. */
int dpa_conv2d_dgrad_fp8(const void* dyq, const void* wq, const float* dy_scale,
                         const float* w_scale, void* dx, void* workspace,
                         int64_t workspace_bytes, int N, int H, int W, int Cin, int Cout,
                         int R, int S, int stride, int pad, void* stream);

/* Same as dpa_conv2d_dgrad_fp8 but takes the weight already transposed to [Cin][R][S][Cout]
 * (as written by dpa_weight_transpose_fp8), so a caller can reuse it across calls. */
int dpa_conv2d_dgrad_fp8_wt(const void* dyq, const void* wq_t, const float* dy_scale,
                            const float* w_scale, void* dx, int N, int H, int W, int Cin,
                            int Cout, int R, int S, int stride, int pad, void* stream);

/* wq_t[Cin][R][S][Cout] = wq[Cout][R][S][Cin] (e4m3 bytes). */
int dpa_weight_transpose_fp8(const void* wq, void* wq_t, int Cout, int R, int S, int Cin,
                             void* stream);

/* Bytes of workspace dpa_conv2d_wgrad_fp8 needs for the given split count
 * (split_k <= 0 selects the library's default for the shape). */
int64_t dpa_conv2d_wgrad_workspace_bytes(int N, int H, int W, int Cin, int Cout, int R,
                                         int S, int stride, int pad, int split_k);

/* dw[Cout,R,S,Cin] = bf16( RN32(sum_splits partial) * RN32(sx * sdy) ),
 * partial[s][co][(r,s,ci)] = sum over output pixels of split s of
 *                            dyq[pix,co] * xq[shifted pix, ci].
 * Splits are summed in index order (deterministic). Replaces
 * conv2d_bwd_weight_fp8_prequantized (diffusion/fp8_kernels.py:723-808), i.e. K7+K8+K9. */
int dpa_conv2d_wgrad_fp8(const void* xq, const void* dyq, const float* x_scale,
                         const float* dy_scale, void* dw, void* workspace,
                         int64_t workspace_bytes, int N, int H, int W, int Cin, int Cout,
                         int R, int S, int stride, int pad, int split_k, void* stream);

/* ------------------------------------------------------------------------------------------
 * FP8 GEMM (the FP8 linear): c[M,N] = bf16( RN32(a[M,K] . b[N,K]^T * RN32(sa*sb)) [+ bias] )
 * a and b are row-major with K contiguous (b is nn.Linear's weight layout).
 * K and N must be multiples of 128. No reference kernel exists (see header comment).
 * ---------------------------------------------------------------------------------------- */
int dpa_gemm_fp8(const void* a, const void* b, const float* a_scale, const float* b_scale,
                 const float* bias, void* c, int M, int N, int K, void* stream);

/* ------------------------------------------------------------------------------------------
 * Split-K variants of the forward conv, the data gradient (pre-transposed weight) and the
 * GEMM. No counterpart in the reference (its kernels launch one program per output tile,
 * diffusion/fp8_kernels.py:624-637 and :694-707); same arguments and results as the entries
 * above up to fp32 summation order. When the output tiles would leave most CUs idle (small
 * images or batches), each tile's K range (taps x channels) is split into equal parts whose
 * fp32 partial sums go to the workspace; a second kernel adds them in split order and
 * applies the same epilogue. The *_split_workspace_bytes queries return the bytes needed
 * (0 when the shape is not split); a workspace of that size must be passed, 16-B aligned.
 * ---------------------------------------------------------------------------------------- */
int64_t dpa_conv2d_fwd_split_workspace_bytes(int N, int H, int W, int Cin, int Cout, int R,
                                             int S, int stride, int pad);
int dpa_conv2d_fwd_fp8_split(const void* xq, const void* wq, const float* x_scale,
                             const float* w_scale, const float* bias, void* y, void* workspace,
                             int64_t workspace_bytes, int N, int H, int W, int Cin, int Cout,
                             int R, int S, int stride, int pad, void* stream);
int64_t dpa_conv2d_dgrad_split_workspace_bytes(int N, int H, int W, int Cin, int Cout, int R,
                                               int S, int stride, int pad);
int dpa_conv2d_dgrad_fp8_wt_split(const void* dyq, const void* wq_t, const float* dy_scale,
                                  const float* w_scale, void* dx, void* workspace,
                                  int64_t workspace_bytes, int N, int H, int W, int Cin,
                                  int Cout, int R, int S, int stride, int pad, void* stream);
int64_t dpa_gemm_split_workspace_bytes(int M, int N, int K);
int dpa_gemm_fp8_split(const void* a, const void* b, const float* a_scale, const float* b_scale,
                       const float* bias, void* c, void* workspace, int64_t workspace_bytes,
                       int M, int N, int K, void* stream);

/* ------------------------------------------------------------------------------------------
 * Fused GroupNorm + optional FiLM + SiLU on NHWC bf16, fp32 statistics (biased variance).
 *   z   = gamma[c] * (x - mean[n,g]) * rstd[n,g] + beta[c]
 *   z'  = film_scale ? film_scale[n,c] * z + film_shift[n,c] : z
 *   out = bf16_RNE( z' * sigmoid(z') )
 * Mirrors F.silu(nn.GroupNorm(G, C)(x)) (diffusion/unet.py:151) and
 * F.silu((w + 1) * nn.GroupNorm(G, C)(x) + b) (diffusion/unet.py:157-159), with
 * film_scale = (w + 1) and film_shift = b given as fp32 [N, C].
 * mean/rstd [N*G] fp32 are written for the backward pass.
 * Requires C % 64 == 0 and 64 % (C / G) == 0 (every GroupNorm of the reference U-Net).
 * ---------------------------------------------------------------------------------------- */
int dpa_gn_silu_fwd_bf16(const void* x, const float* gamma, const float* beta,
                         const float* film_scale, const float* film_shift, void* out,
                         float* mean, float* rstd, int N, int HW, int C, int G, float eps,
                         void* stream);

/* The same forward with a workspace (size from dpa_gn_silu_fwd_workspace_bytes: 0 under 256
 * pixels; nonzero from 256, used only above 1024). Which form runs, by image size HW:
 *   HW <= 1024: the resident form, one launch, one workgroup per (image, 64-channel slab)
 *     holding the slab's pixels in registers (no workspace read);
 *   1024 < HW <= 8192 with the workspace: the chunked form, two launches, each (image, slab)
 *     spread over workgroups of 128 pixels whose group statistics (chunk mean and squared
 *     deviations, merged in chunk order) cross through the workspace;
 *   otherwise (HW > 8192, or no workspace): one launch of one workgroup per (image, slab)
 *     making three passes over the slab.
 * The FiLM is either film_scale/film_shift (fp32 [N, C]) or film_wb (the bf16 time
 * projection [N, 2C], as in dpa_gn_silu_film_fwd_bf16) or neither. */
int64_t dpa_gn_silu_fwd_workspace_bytes(int N, int HW, int C, int G);
int dpa_gn_silu_fwd_ws_bf16(const void* x, const float* gamma, const float* beta,
                            const float* film_scale, const float* film_shift, const void* film_wb,
                            void* out, float* mean, float* rstd, void* workspace,
                            int64_t workspace_bytes, int N, int HW, int C, int G, float eps,
                            void* stream);

/* Bytes of workspace dpa_gn_silu_bwd_bf16 needs: per-image channel partial sums (2*N*C fp32)
 * and, from 256 pixels, room for the chunk sums of the chunked backward (two launches like
 * the forward). The backward runs the resident form up to 1024 pixels (fp32 x with FiLM or
 * dropout: up to 256 pixels, since x, the FiLM terms and the keep bits exceed the register
 * file at 16 pixels per lane), the chunked form above that up to 8192 pixels with the full
 * workspace, and the one-launch form with a workspace of only 2*N*C floats. */
int64_t dpa_gn_silu_bwd_workspace_bytes(int N, int HW, int C, int G);

/* Backward of dpa_gn_silu_fwd_bf16 given dout (bf16, same layout as out). Writes dx (bf16)
 * and overwrites dgamma, dbeta [C] and, when film_scale is given, dfilm_scale and
 * dfilm_shift [N, C] (all fp32). Per-channel sums over the batch are reduced in image
 * order (deterministic). */
int dpa_gn_silu_bwd_bf16(const void* x, const void* dout, const float* gamma,
                         const float* beta, const float* film_scale, const float* film_shift,
                         const float* mean, const float* rstd, void* dx, float* dgamma,
                         float* dbeta, float* dfilm_scale, float* dfilm_shift, void* workspace,
                         int64_t workspace_bytes, int N, int HW, int C, int G, void* stream);

/* dpa_gn_silu_fwd_bf16 / _bwd with the FiLM taken straight from the bf16 time projection
 * film_wb [N, 2C] of diffusion/unet.py:157-158 (w = film_wb[:, :C], b = film_wb[:, C:]):
 * scale bf16(w + 1) (the reference's bf16 add), shift b. The backward writes the gradient of
 * film_wb [N, 2C] in bf16 (the reference's chunk/add/dtype-cast backward, in place of three
 * more launches). */
int dpa_gn_silu_film_fwd_bf16(const void* x, const float* gamma, const float* beta,
                              const void* film_wb, void* out, float* mean, float* rstd, int N,
                              int HW, int C, int G, float eps, void* stream);
int dpa_gn_silu_film_bwd_bf16(const void* x, const void* dout, const float* gamma,
                              const float* beta, const void* film_wb, const float* mean,
                              const float* rstd, void* dx, float* dgamma, float* dbeta,
                              void* dfilm_wb, void* workspace, int64_t workspace_bytes, int N,
                              int HW, int C, int G, void* stream);

/* Element type of x (and dx) for the *_ex GroupNorm entries. */
#define DPA_DTYPE_BF16 0
#define DPA_DTYPE_F32 1

/* GroupNorm + FiLM + SiLU forward / backward with x (and dx) in bf16 or fp32, the other
 * arguments as in dpa_gn_silu_fwd_ws_bf16 / dpa_gn_silu_bwd_bf16 (one FiLM form at a time:
 * film_scale/film_shift or film_wb). Under autocast the reference normalises an fp32 input
 * in fp32 (nn.GroupNorm runs in float32, diffusion/unet.py:151, :157) and returns an fp32
 * input gradient; with DPA_DTYPE_F32 the kernels read the fp32 x as it is and write dx in
 * fp32 (the output y stays bf16). fp32 x takes the resident form (images of up to 1024
 * pixels; the backward with FiLM or dropout up to 256) or the chunked form (above that, up to
 * 8192 pixels, with a workspace of the *_workspace_bytes size); larger images return
 * DPA_ERR_SHAPE, a missing workspace DPA_ERR_WORKSPACE.
 * Optional dropout of the output (diffusion/unet.py:160, nn.Dropout(p) before conv_2):
 * drop_seed = a uint64 in device memory, NULL for none; an element is kept when bits
 * [16 (idx % 4), 16 (idx % 4) + 16) of splitmix64(seed + (idx / 4) * 0x9E3779B97F4A7C15)
 * (idx its NHWC index), as a 16-bit number, are >= floor(p * 2^16) with p the fp32 drop_p
 * argument (exact in double), and kept values are
 * scaled in fp32 by RN32(1 / RN32(1 - p)) before the bf16 rounding (the
 * reference drops the fp32 SiLU output). The backward recomputes the mask from the same seed
 * and p. Dropout takes the resident or chunked form as fp32 x does; 0 <= p < 1.
 * dx_add (backward; x's dtype and layout, or NULL): a second gradient of x added to dx as
 * autograd accumulates it (fp32: one add; bf16: bf16(dx) + add, rounded to bf16) — the skip
 * path's gradient of the residual block input (diffusion/unet.py:149, :161), which x feeds
 * besides norm1; dx_add_dtype DPA_DTYPE_BF16 with an fp32 x adds a bf16 gradient (autograd's
 * fp32 cast of it, then one fp32 add). Resident or chunked form only; may alias dx.
 * Any other dx_add_dtype, or an fp32 dx_add beside a bf16 x, returns DPA_ERR_SHAPE.
 * x_bf16 (forward, fp32 x only, or NULL): also writes x rounded to bf16 (RNE) there — the
 * input the 1x1 skip conv rounds to anyway — so no separate cast pass reads x again. */
int dpa_gn_silu_fwd_ex(const void* x, int x_dtype, const float* gamma, const float* beta,
                       const float* film_scale, const float* film_shift, const void* film_wb,
                       void* out, float* mean, float* rstd, void* workspace,
                       int64_t workspace_bytes, int N, int HW, int C, int G, float eps,
                       const void* drop_seed, float drop_p, void* x_bf16, void* stream);
int dpa_gn_silu_bwd_ex(const void* x, int x_dtype, const void* dout, const float* gamma,
                       const float* beta, const float* film_scale, const float* film_shift,
                       const void* film_wb, const float* mean, const float* rstd, void* dx,
                       const void* dx_add, int dx_add_dtype, float* dgamma, float* dbeta,
                       float* dfilm_scale,
                       float* dfilm_shift, void* dfilm_wb, void* workspace,
                       int64_t workspace_bytes, int N, int HW, int C, int G, const void* drop_seed, float drop_p, void* stream);

/* Producer-fused quantization for a delayed-scaling FP8 conv. Replaces the conv's separate
 * input cast (diffusion/fp8_kernels.py:856, quantize_fp8_delayed at :518-556 with its
 * partial_amax_kernel_delayed :69-87) after the GroupNorm+SiLU producers of
 * diffusion/unet.py:151 and :157-160, and its dy cast (:885-893) after the GroupNorm
 * backward that produces conv_1's dy. In delayed scaling the scale is the window's, known
 * before the producer runs, so the producer writes the conv operand directly:
 *   q = e4m3(clamp(bf16 value / *q_scale))   (the bf16-then-e4m3 double rounding)
 * instead of the bf16 output (fwd) or bf16 dx (bwd), and each workgroup stores the amax of
 * its bf16 values as bf16 magnitude bits in q_partials[workgroup], workgroup 0 the count in
 * *q_count: the layout dpa_quantize_fp8_delayed_deferred_bf16 leaves for
 * dpa_delayed_windows_finalize. Bytes and window record equal those of the unfused pair
 * (bf16 entry, then the deferred cast). Arguments otherwise as dpa_gn_silu_fwd_ex /
 * dpa_gn_silu_bwd_ex; the backward takes bf16 x and no dx_add. The resident form (images of
 * up to 1024 pixels, one partial per (image, 64-channel slab)) and the chunked form (up to
 * 8192 pixels with the workspace, one partial per 128-pixel chunk of each slab) cast; larger
 * images return DPA_ERR_SHAPE, a chunked-size image without the workspace
 * DPA_ERR_WORKSPACE. q_partials_cap < dpa_gn_silu_fp8_partials(...) returns
 * DPA_ERR_WORKSPACE. */
int dpa_gn_silu_fp8_partials(int N, int HW, int C, int G);
int dpa_gn_silu_fwd_fp8(const void* x, int x_dtype, const float* gamma, const float* beta,
                        const float* film_scale, const float* film_shift, const void* film_wb,
                        void* q, const float* q_scale, uint32_t* q_partials, int q_partials_cap,
                        uint32_t* q_count, float* mean, float* rstd, void* workspace,
                        int64_t workspace_bytes, int N, int HW, int C, int G, float eps,
                        const void* drop_seed, float drop_p, void* x_bf16, void* stream);

/* dpa_gn_silu_fwd_ex / dpa_gn_silu_fwd_fp8 that also leave, with x_bf16 (fp32 x), one amax
 * partial of the bf16 copy of x per workgroup of the launch that writes it (u32 bf16
 * magnitude bits; count dpa_gn_silu_fp8_partials(N, HW, C, G)): the copy is the input of the
 * residual block's 1x1 skip conv (diffusion/unet.py:137-139, :161), which quantizes it with
 * current scaling, and dpa_quantize_fp8_bf16_from_partials takes these partials in place of
 * its amax pass (partial_amax_kernel, diffusion/fp8_kernels.py:54-64). Resident and chunked
 * forms; xb_partials_cap below the count returns DPA_ERR_WORKSPACE. */
int dpa_gn_silu_fwd_ex_amax(const void* x, int x_dtype, const float* gamma, const float* beta,
                            const float* film_scale, const float* film_shift,
                            const void* film_wb, void* out, float* mean, float* rstd,
                            void* workspace, int64_t workspace_bytes, int N, int HW, int C,
                            int G, float eps, const void* drop_seed, float drop_p,
                            void* x_bf16, uint32_t* xb_partials, int xb_partials_cap,
                            void* stream);
int dpa_gn_silu_fwd_fp8_amax(const void* x, int x_dtype, const float* gamma, const float* beta,
                             const float* film_scale, const float* film_shift,
                             const void* film_wb, void* q, const float* q_scale,
                             uint32_t* q_partials, int q_partials_cap, uint32_t* q_count,
                             float* mean, float* rstd, void* workspace, int64_t workspace_bytes,
                             int N, int HW, int C, int G, float eps, const void* drop_seed,
                             float drop_p, void* x_bf16, uint32_t* xb_partials,
                             int xb_partials_cap, void* stream);
int dpa_gn_silu_bwd_fp8(const void* x, const void* dout, const float* gamma, const float* beta,
                        const float* film_scale, const float* film_shift, const void* film_wb,
                        const float* mean, const float* rstd, void* dxq, const float* dx_scale,
                        uint32_t* dx_partials, int dx_partials_cap, uint32_t* dx_count,
                        float* dgamma, float* dbeta, float* dfilm_scale, float* dfilm_shift,
                        void* dfilm_wb, void* workspace, int64_t workspace_bytes, int N, int HW,
                        int C, int G, const void* drop_seed, float drop_p, void* stream);

/* ------------------------------------------------------------------------------------------
 * Grouped FP8 weight preparation. No single counterpart in the reference: it performs, for a
 * model's whole FP8 weight set in three launches per step, what the reference does per layer
 * call (autocast bf16 cast of the fp32 weight, quantize_fp8 / quantize_fp8_delayed of
 * diffusion/fp8_kernels.py:518-601, the amax-window updates of diffusion/unet.py:69-91, and
 * the weight transpose the data gradient needs). Bytes and scales are identical to the
 * per-layer path: bf16(w) is the round-to-nearest-even cast, then the same scale and e4m3
 * rule as dpa_quantize_fp8_bf16 (current scaling) or dpa_quantize_fp8_delayed_bf16 (delayed).
 * ---------------------------------------------------------------------------------------- */
#define DPA_WP_BF16 1          /* DpaWeightEntry.flags: w holds bf16, not fp32 */
#define DPA_WP_FRAG 2          /* q and qt in the fragment layouts of dpa_weight_frag_fp8
                                  (forward / data gradient); Cin, Cout multiples of 128 */
typedef struct DpaWeightEntry {
  const float* w;           /* weight (fp32, or bf16 with DPA_WP_BF16), FP8 memory order:
                               [Cout][R][S][Cin] or [N][K] */
  void* q;                  /* e4m3 out, same order (8-B aligned) */
  void* qt;                 /* e4m3 out [Cin][R][S][Cout] (data-gradient operand) or NULL */
  float* scale_used;        /* the scale q was cast with */
  float* cur_scale;         /* scale of this weight's own amax, or NULL */
  const float* prev_scale;  /* delayed scaling: the scale to cast with; NULL: current */
  float* window;            /* delayed: amax window, cur_scale recorded at *pos, or NULL */
  int64_t* pos;             /*   (pos itself is not advanced) */
  int64_t window_len;
  int64_t n;                /* elements = cout * taps * cin (cin % 8 == 0) */
  int32_t cout, taps, cin;  /* taps = R * S (1 for a linear) */
  int32_t blk0, nblk;       /* filled in by dpa_weight_prep_plan */
  int32_t flags;            /* DPA_WP_BF16 | DPA_WP_FRAG, or 0 */
} DpaWeightEntry;

/* Assigns each entry its blocks (host array, in place); returns the total block count (> 0)
 * or a negative status. Copy the planned array to device memory for dpa_weight_prep_run. */
int dpa_weight_prep_plan(DpaWeightEntry* entries, int count);
int64_t dpa_weight_prep_workspace_bytes(int total_blocks);
/* Two launches: per-block amax of bf16(w), then cast + transposed cast + scales + window
 * records. Entries whose prev_scale points at dpa_window_max_grouped_f32 output must follow
 * that call on the same stream. */
int dpa_weight_prep_run(const DpaWeightEntry* entries_dev, int count, int total_blocks,
                        void* workspace, int64_t workspace_bytes, void* stream);
/* dpa_quantize_fp8_bf16(x, ...) and dpa_weight_prep_run(entries_dev, ...) in two launches
 * instead of four: the preparation's blocks run inside x's amax and cast launches, with the
 * same results as the two calls. For a caller that quantizes an activation and prepares a
 * weight for the same GEMM, as the reference's conv2d_fwd_fp8 (diffusion/fp8_kernels.py:
 * 642-650) quantizes x and the weight one after the other (quantize_fp8 :559-601 twice). */
int dpa_quantize_fp8_bf16_with_weight_prep(const void* x, int64_t n, void* q, float* scale_out,
                                           void* workspace, int64_t workspace_bytes,
                                           const DpaWeightEntry* entries_dev, int count,
                                           int total_blocks, void* wp_workspace,
                                           int64_t wp_workspace_bytes, void* stream);
/* hist[i] = max over window i of len floats (torch.max; NaN if the window holds one);
 * windows_dev: device array of count window pointers. One launch for every window. */
int dpa_window_max_grouped_f32(const float* const* windows_dev, int count, int64_t len,
                               float* hist, void* stream);

/* Deferred window records for layers whose weights are prepared per step. No counterpart in
 * the reference (which records each scale in its own finalize, diffusion/fp8_kernels.py:
 * 90-102, and the module's scatter_, diffusion/unet.py:82-91): the x and dy quantizations of
 * a delayed-scaling layer cast with their window scale (as dpa_quantize_fp8_delayed_bf16) and
 * leave their block maxima and count in caller-owned persistent buffers; one launch at the
 * start of the next step writes every layer's records (window_acts[pos] from x,
 * window_dy[pos + 1] from dy, pos + 1 if x was quantized), which is the window state the
 * per-call path leaves after the step. Counts must be zero before the first use; the
 * finalize sets them back to zero. */
typedef struct DpaDeferredWindow {
  const uint32_t* x_partials;   /* >= dpa_quant_partials_count(numel(x)) u32 */
  uint32_t* x_count;
  const uint32_t* dy_partials;
  uint32_t* dy_count;
  float* window_acts;
  float* window_dy;
  int64_t* pos;
  int64_t len;
} DpaDeferredWindow;

int dpa_quant_partials_count(int64_t n);
int dpa_quantize_fp8_delayed_deferred_bf16(const void* x, int64_t n, const float* prev_scale,
                                           void* q, uint32_t* partials, int partials_cap,
                                           uint32_t* count, void* stream);
int dpa_delayed_windows_finalize(const DpaDeferredWindow* layers_dev, int count, void* stream);

/* dpa_conv2d_wgrad_fp8 writing fp32 dw holding the bf16-rounded values (what autograd's cast
 * of the reference's bf16 gradient to an fp32 parameter produces), in the same
 * [Cout][R][S][Cin] order: the gradient of a channels-last fp32 master weight directly. */
int dpa_conv2d_wgrad_fp8_f32(const void* xq, const void* dyq, const float* x_scale,
                             const float* dy_scale, float* dw, void* workspace,
                             int64_t workspace_bytes, int N, int H, int W, int Cin, int Cout,
                             int R, int S, int stride, int pad, int split_k, void* stream);

/* ------------------------------------------------------------------------------------------
 * Grouped FP8 linear layers over one shared input x [M][K]: the FiLM projections of the U-Net's
 * residual blocks (diffusion/unet.py:101-104, :135 -- every block's Linear(512, 2C) reads the
 * same time embedding). No single counterpart in the reference (its Linears run per layer);
 * per layer i (n_i output features) the arithmetic is the per-layer FP8 recipe with the
 * layer's own per-tensor scales, one launch for all layers per direction:
 *   quantize: q_i = e4m3(src_i / s_i), s_i = amax(src_i) > 0 ? RN32(amax / 448) : 1, as
 *             dpa_quantize_fp8_bf16 (bytes and scales identical), written into one
 *             concatenated [R][sum n_i] buffer q and/or its transpose qt [sum n_i][R];
 *   forward:  y_i = bf16(RN32(acc * RN32(s_x s_wi))), y_i [M][n_i], w_i [n_i][K] e4m3;
 *   wgrad:    dw_i = bf16(RN32(acc * RN32(s_x s_dyi))) stored as fp32 [n_i][K], from the
 *             transposes xq_t [K][M] and dyq_t [sum n_i][M];
 *   dgrad:    dx = bf16(sum_i RN32(acc_i * RN32(s_dyi s_wi))), the layers summed in fp32 in
 *             order, from dyq [M][sum n_i] and the transposed weights w_i^T [K][n_i].
 * At most 32 layers; n_i % 64 == 0 (dgrad: % 128), M % 64 == 0 (wgrad: % 128), K % 128 == 0.
 * ---------------------------------------------------------------------------------------- */
int dpa_grouped_quantize_fp8_bf16(const void* const* src, const int* n, int nseg, int R,
                                  void* q, void* qt, float* scale, void* stream);
int dpa_grouped_linear_fwd_fp8(const void* xq, const float* x_scale, const void* const* wq,
                               const float* const* w_scale, void* const* y, const int* n,
                               int nseg, int M, int K, void* stream);
int dpa_grouped_linear_wgrad_fp8_f32(const void* xq_t, const float* x_scale, const void* dyq_t,
                                     const float* dy_scale, float* const* dw, const int* n,
                                     int nseg, int M, int K, void* stream);
int64_t dpa_grouped_linear_dgrad_workspace_bytes(int nseg, int M, int K);
int dpa_grouped_linear_dgrad_fp8(const void* dyq, const float* dy_scale, const void* const* wq_t,
                                 const float* const* w_scale, void* dx, const int* n, int nseg,
                                 int M, int K, void* workspace, int64_t workspace_bytes,
                                 void* stream);

/* ------------------------------------------------------------------------------------------
 * LayerNorm over the channel axis of bf16 token rows [rows][C], fp32 statistics (biased
 * variance), bf16 out: the attention block's nn.LayerNorm (diffusion/unet.py:174, applied at
 * :187 to the [B, H*W, C] view of the channels-last activation; autocast runs it in fp32 and
 * the qkv projection rounds its output to bf16, which is what `out` stores).
 *   out = bf16((x - mean) * rstd * gamma + beta);  mean/rstd [rows] saved for the backward.
 * Backward: dx (bf16), dgamma/dbeta (fp32, summed over rows in a fixed order).
 * C % 64 == 0 with C / 64 in {1, 2, 4, 8, 16}.
 * ---------------------------------------------------------------------------------------- */
int dpa_layernorm_fwd_bf16(const void* x, const float* gamma, const float* beta, void* out,
                           float* mean, float* rstd, int64_t rows, int C, float eps,
                           void* stream);
int64_t dpa_layernorm_bwd_workspace_bytes(int64_t rows, int C);
int dpa_layernorm_bwd_bf16(const void* x, const void* dout, const float* gamma,
                           const float* mean, const float* rstd, void* dx, float* dgamma,
                           float* dbeta, void* workspace, int64_t workspace_bytes, int64_t rows,
                           int C, void* stream);

/* The LayerNorm entries with x (and dx) in bf16 or fp32 (DPA_DTYPE_*), the output y bf16:
 * an fp32 token row (the fp32 residual stream) is normalised as it is, as autocast's float32
 * nn.LayerNorm does (diffusion/unet.py:174, :187), and its gradient returned in fp32. */
int dpa_layernorm_fwd_ex(const void* x, int x_dtype, const float* gamma, const float* beta,
                         void* out, float* mean, float* rstd, int64_t rows, int C, float eps,
                         void* stream);
int dpa_layernorm_bwd_ex(const void* x, int x_dtype, const void* dout, const float* gamma,
                         const float* mean, const float* rstd, void* dx, float* dgamma,
                         float* dbeta, void* workspace, int64_t workspace_bytes, int64_t rows,
                         int C, void* stream);
/* The backward with the gradient the attention block's skip path gives the same tokens
 * (dx_add, x's dtype, 16-B aligned) added to dx as it is stored, as autograd adds the two
 * gradients of the block input (diffusion/unet.py:182-187, :201: x feeds the LayerNorm and
 * the residual join): fp32 + fp32, or bf16(dx) + dx_add in fp32 rounded to bf16. */
int dpa_layernorm_bwd_ex_add(const void* x, int x_dtype, const void* dout, const float* gamma,
                             const float* mean, const float* rstd, const void* dx_add, void* dx,
                             float* dgamma, float* dbeta, void* workspace,
                             int64_t workspace_bytes, int64_t rows, int C, void* stream);

/* The forward also writing the per-workgroup maxima of |y| (bf16 magnitude bits) to
 * amax_partials (dpa_layernorm_fwd_partials(rows, C) entries; 0 for an unsupported shape),
 * for the qkv projection's current-scaling cast (dpa_quantize_fp8_bf16_from_partials) in
 * place of its amax pass (partial_amax_kernel, diffusion/fp8_kernels.py:54-64). */
int dpa_layernorm_fwd_partials(int64_t rows, int C);
int dpa_layernorm_fwd_amax(const void* x, int x_dtype, const float* gamma, const float* beta,
                           void* out, float* mean, float* rstd, int64_t rows, int C, float eps,
                           void* amax_partials, void* stream);

/* ------------------------------------------------------------------------------------------
 * Self-attention of the attention block, softmax(q k^T / sqrt(64)) v per (image, head), bf16
 * in and out, fp32 softmax: replaces F.scaled_dot_product_attention with its head rearranges
 * (diffusion/unet.py:188-198): q, k, v are read in place from the qkv projection's output
 * qkv [B][L][3C] (q = columns [0, C), k = [C, 2C), v = [2C, 3C), head h at h*64 of each),
 * the output is written as out [B][L][C] ("b nh l hd -> b l (nh hd)"), and
 * lse [B*heads][L] (fp32, base-2 log-sum-exp of the scaled scores) is kept for the backward.
 * Backward: dout [B][L][C] -> dqkv [B][L][3C] (dq, dk, dv in the qkv layout), recomputing the
 * probabilities from lse. Deterministic (no atomics).
 * C == 64 * heads; L % 16 == 0, 16 <= L <= 256 (the U-Net's 16x16, 8x8 and 4x4 token grids);
 * qkv, out (backward), dout 16-B aligned; out (forward) and dqkv 8-B aligned.
 * ---------------------------------------------------------------------------------------- */
int dpa_attention_fwd_bf16(const void* qkv, void* out, float* lse, int B, int L, int C,
                           int heads, void* stream);
int dpa_attention_bwd_bf16(const void* qkv, const void* out, const void* dout,
                           const float* lse, void* dqkv, int B, int L, int C, int heads,
                           void* stream);

/* The same with one amax partial per (image, head) workgroup, B * heads of them, in
 * amax_partials: the max |out| (forward) or |dqkv| (backward) as bf16 magnitude bits, for the
 * current-scaling cast of the out projection's input and of the qkv projection's output
 * gradient (dpa_quantize_fp8_bf16_from_partials) in place of their amax passes
 * (partial_amax_kernel, diffusion/fp8_kernels.py:54-64). */
int dpa_attention_fwd_amax(const void* qkv, void* out, float* lse, int B, int L, int C,
                           int heads, void* amax_partials, void* stream);
int dpa_attention_bwd_amax(const void* qkv, const void* out, const void* dout,
                           const float* lse, void* dqkv, int B, int L, int C, int heads,
                           void* amax_partials, void* stream);

/* Residual join y = (a + b) / sqrt(2) of bf16 tensors in one pass (diffusion/unet.py:161 and
 * :203, under autocast), with torch's roundings: bf16(bf16(a + b) * inv), inv = RN32(1/sqrt 2)
 * passed by the caller. b == NULL gives y = bf16(a * inv) (the backward). n % 8 == 0,
 * pointers 16-B aligned, same memory order for a, b and y. */
int dpa_residual_scale_bf16(const void* a, const void* b, void* y, int64_t n, float inv,
                            void* stream);

/* The same join on the fp32 residual stream: a fp32, b bf16 (the branch output), y fp32 =
 * RN32(RN32(a + b) * inv), torch's (a + b) / math.sqrt(2.0) with type promotion
 * (diffusion/unet.py:161, :203 below the first level, where the skip path is fp32 under
 * autocast). n % 4 == 0; a, y 16-B and b 8-B aligned. */
int dpa_residual_scale_f32(const float* a, const void* b, float* y, int64_t n, float inv,
                           void* stream);
/* Its backward: ga = g * inv (fp32), gb = bf16(g * inv), one pass over g. */
int dpa_residual_scale_bwd_f32(const float* g, float* ga, void* gb, int64_t n, float inv,
                               void* stream);
/* The join's backward when b is the output of a delayed-scaling FP8 conv (the conv_2 of
 * diffusion/unet.py:160-161): b's gradient bf16(g * inv) is cast for that conv instead of
 * stored -- gbq = e4m3(clamp(gb / *gb_scale)) with one amax partial per workgroup, as the
 * fused GroupNorm entries above (replacing the conv's dy cast, diffusion/fp8_kernels.py:
 * 885-893) -- and ga is stored as in the plain backward: fp32 g * inv for an fp32 g
 * (g_dtype DPA_DTYPE_F32, the dpa_residual_scale_bwd_f32 form) or the bf16 values
 * bf16(g * inv) for a bf16 g (the backward of dpa_residual_scale_bf16). n % 8 == 0;
 * gb_partials_cap >= dpa_residual_scale_fp8_partials(n). */
int dpa_residual_scale_fp8_partials(int64_t n);
int dpa_residual_scale_bwd_fp8(const void* g, int g_dtype, void* ga, void* gbq,
                               const float* gb_scale, uint32_t* gb_partials, int gb_partials_cap,
                               uint32_t* gb_count, int64_t n, float inv, void* stream);

/* The join's backward when the bf16 gradient it writes is quantized next by a current-scaling
 * FP8 GEMM (the attention out-projection of diffusion/unet.py:199-203, a 1x1 skip conv or a
 * current-scaling conv feeding the join): the plain backward (g_dtype DPA_DTYPE_F32: ga = g * inv
 * in fp32 and gb = bf16(g * inv), as dpa_residual_scale_bwd_f32; DPA_DTYPE_BF16: ga NULL and
 * gb = bf16(g * inv), the one gradient both operands receive, as dpa_residual_scale_bf16 with
 * b NULL) plus one amax partial of gb per workgroup (u32 bf16 magnitude bits; count
 * dpa_residual_scale_fp8_partials(n)), which dpa_quantize_fp8_bf16_from_partials takes in place
 * of the quantization's amax pass (partial_amax_kernel, diffusion/fp8_kernels.py:54-64).
 * n % 8 == 0, g, ga, gb 16-B aligned. */
int dpa_residual_scale_bwd_amax(const void* g, int g_dtype, float* ga, void* gb,
                                uint32_t* gb_partials, int gb_partials_cap, int64_t n,
                                float inv, void* stream);

/* Decoder input of the U-Net: y = cat([up(a), h], dim=1) in NHWC, fp32, where up is the 2x
 * nearest upsampling (up = 1) or the identity (up = 0) -- diffusion/unet.py:379-382,
 * torch.concat([self.upsample(act), h]) under autocast (F.interpolate runs in fp32 and the
 * concatenation promotes). a: [N][H >> up][W >> up][C1], h: [N][H][W][C2], each bf16 or fp32
 * (DPA_DTYPE_*); y: [N][H][W][C1 + C2] fp32. C1, C2 multiples of 4. One pass, no upsampled
 * intermediate. */
int dpa_upsample_concat_f32(const void* a, int a_dtype, const void* h, int h_dtype, float* y,
                            int N, int H, int W, int C1, int C2, int up, void* stream);
/* Its backward from gy (fp32, y's shape): ga = the sum of gy over each up x up window
 * (accumulated from zero in row-major order, as torch's upsample_nearest2d_backward), gh =
 * gy's last C2 channels, each in its operand's dtype. */
int dpa_upsample_concat_bwd_f32(const float* gy, void* ga, int a_dtype, void* gh, int h_dtype,
                                int N, int H, int W, int C1, int C2, int up, void* stream);

/* A decoder stage's first GroupNorm+SiLU with the upsample-and-concatenate before it
 * (diffusion/unet.py:379-382 with :151; no counterpart op in the reference): x =
 * cat([up2(a), h], channels) read from a ([N][H/2][W/2][Ca], bf16) and h ([N][H][W][Ch],
 * h_dtype: DPA_DTYPE_BF16, or DPA_DTYPE_F32 at 16x16), NHWC, instead of from the fp32
 * concatenation (which holds exactly those values), so neither the concatenation nor its
 * gradient is written. Outputs as dpa_gn_silu_fwd_fp8_amax for an fp32 x: out (bf16
 * [N][H][W][C], C = Ca + Ch) or, instead, the e4m3 hand-off q (q_scale, q_partials, q_count
 * as there); x_bf16 (optional) the bf16 concatenation, with one amax partial per workgroup in
 * xb_partials (optional); mean / rstd [N][G]. H = W = 32 (h bf16) or 16, Ca and Ch multiples
 * of 64; no FiLM, no dropout. Bit-identical to dpa_upsample_concat_f32 followed by the
 * GroupNorm on its fp32 result. */
int dpa_upcat_gn_silu_fwd(const void* a, const void* h, int h_dtype, int N, int H, int W,
                          int Ca, int Ch, const float* gamma, const float* beta, void* out,
                          void* q, const float* q_scale, uint32_t* q_partials,
                          int q_partials_cap, uint32_t* q_count, float* mean, float* rstd,
                          void* x_bf16, uint32_t* xb_partials, int xb_partials_cap, int G,
                          float eps, void* stream);
/* Its backward: the concatenation's gradient (the GroupNorm's fp32 dx plus dx_add, a bf16
 * gradient of the concatenation from its other reader, the 1x1 skip conv, or NULL) goes
 * straight to ga (bf16, a's shape: each 2x2 window summed from zero in row-major order) and
 * gh (h's dtype and shape), as dpa_upsample_concat_bwd_f32 splits it; dgamma, dbeta as
 * dpa_gn_silu_bwd_ex (workspace of 2 N C floats). */
int dpa_upcat_gn_silu_bwd(const void* a, const void* h, int h_dtype, int N, int H, int W,
                          int Ca, int Ch, const void* dout, const float* gamma,
                          const float* beta, const float* mean, const float* rstd,
                          const void* dx_add, void* ga, void* gh, float* dgamma, float* dbeta,
                          void* workspace, int64_t workspace_bytes, int G, void* stream);

/* Encoder downsampling F.interpolate(a, scale_factor=0.5, mode="nearest") under autocast
 * (diffusion/unet.py:370-373): y[n][i][j][c] = a[n][2i][2j][c] as fp32; a [N][H][W][C] bf16
 * or fp32 (H, W even, C % 4 == 0), y [N][H/2][W/2][C]. The backward writes ga (a's dtype and
 * shape): gy at the sampled pixels, 0 elsewhere. One pass each. */
int dpa_downsample2_f32(const void* a, int a_dtype, float* y, int N, int H, int W, int C,
                        void* stream);
int dpa_downsample2_bwd_f32(const float* gy, void* ga, int a_dtype, int N, int H, int W, int C,
                            void* stream);
/* The backward when a has a second reader whose gradient gskip (a's dtype and shape) is
 * ready (the encoder activation that the decoder's concatenation also reads,
 * diffusion/unet.py:363-376): ga = a_dtype(gy at the sampled pixels, 0 elsewhere) + gskip, one
 * add in a's dtype as autograd accumulates the two gradients; one pass instead of the
 * backward plus autograd's add. ga may alias gskip. */
int dpa_downsample2_bwd_add_f32(const float* gy, const void* gskip, void* ga, int a_dtype, int N,
                                int H, int W, int C, void* stream);

/* The training loss mean((pred - target)^2) of the DDPM step (diffusion/ddpm.py:209-215,
 * F.mse_loss with both operands in fp32 under autocast): pred bf16 or fp32 (DPA_DTYPE_*),
 * target fp32, same memory order, n elements; *out = fp32 loss. Deterministic (fixed-order
 * partial sums in the workspace, then one workgroup), two launches, nothing cleared by a
 * memset -- safe inside a captured HIP graph. */
int64_t dpa_mse_loss_workspace_bytes(void);
int dpa_mse_loss_f32(const void* pred, int pred_dtype, const float* target, int64_t n,
                     float* out, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * Optimizer tail of the training step (train.py:104-149): clip_grad_norm_(max_norm),
 * AdamW (torch.optim.AdamW, :253: betas, eps, weight_decay) and the EMA update (:256,
 * ddpm.py EWMAWrapper.update) in one gradient-norm pass and one update pass over all
 * tensors. Entries with a grad get the clipped AdamW update and then, if ema is set,
 * ema = RN(beta ema) + RN((1 - beta) p); entries without a grad (float buffers) only the EMA.
 * The global norm is sqrt(sum of fixed-range block sums, in order): deterministic. *step is
 * the device step count (incremented here, as the capturable optimizer's). All pointers
 * fp32, 16-B aligned; the tensors array is host memory (pointers go in kernel arguments).
 * No counterpart entry in the reference (three library calls there).
 * ---------------------------------------------------------------------------------------- */
typedef struct DpaOptTensor {
  float* param;
  const float* grad;   /* NULL: EMA-only entry */
  float* exp_avg;
  float* exp_avg_sq;
  float* ema;          /* NULL: no EMA copy */
  int64_t n;
} DpaOptTensor;

int64_t dpa_adamw_ema_workspace_bytes(const DpaOptTensor* tensors, int count);
int dpa_adamw_ema_step(const DpaOptTensor* tensors, int count, float* step, float lr,
                       float beta1, float beta2, float eps, float weight_decay, float max_norm,
                       float ema_beta, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------------------------
 * bf16 3x3 / stride-1 / pad-1 convolutions with an image-channel side: the U-Net's input conv
 * (diffusion/unet.py:255-257, nn.Conv2d(3, C, 3, padding=1, bias=False)) and its output head's
 * conv (:325-329, nn.Conv2d(C, 3, ...)), which the reference runs in bf16 under autocast
 * (train.py:120, :136): bf16 operands, fp32 accumulation, bf16 output. One side has 1-3
 * channels, the other 128 or 256; NHWC activations, W in {16, 32, 64}, H a multiple of
 * 64 / W; the weight [Cout][Cin][3][3] fp32 or bf16 (w_dtype) at element strides ws0..ws3,
 * rounded to bf16 on load. Other shapes return DPA_ERR_SHAPE. No counterpart entry in the
 * reference (cuDNN through nn.Conv2d there).
 * fwd: x bf16, or for a thin input fp32 (rounded to bf16 on load, as autocast's cast);
 * y bf16 [N][H][W][Cout], 16-B aligned.
 * dgrad: Cout <= 3 only (dy thin, bf16): dx bf16 [N][H][W][Cin].
 * wgrad: dw fp32 [Cout][3][3][Cin] = fp32(bf16(sum over pixels)) -- the bf16 weight gradient
 * cast back to the fp32 weight, as autocast's; partial sums per workgroup in the workspace
 * (dpa_conv3x3_thin_wgrad_workspace_bytes), added in a fixed order: deterministic. */
int dpa_conv3x3_thin_fwd(const void* x, int x_dtype, const void* w, int w_dtype, int ws0,
                         int ws1, int ws2, int ws3, void* y, int N, int H, int W, int Cin,
                         int Cout, void* stream);
int dpa_conv3x3_thin_dgrad(const void* dy, const void* w, int w_dtype, int ws0, int ws1,
                           int ws2, int ws3, void* dx, int N, int H, int W, int Cin, int Cout,
                           void* stream);
int64_t dpa_conv3x3_thin_wgrad_workspace_bytes(int N, int H, int W, int Cin, int Cout);
int dpa_conv3x3_thin_wgrad(const void* x, int x_dtype, const void* dy, float* dw, int N, int H,
                           int W, int Cin, int Cout, void* workspace, int64_t workspace_bytes,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DPA_FP8_H */
