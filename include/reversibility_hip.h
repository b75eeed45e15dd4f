/*
 * reversibility_hip.h -- C ABI of the MI355X (gfx950) kernels behind the
 * reversible-training hot path: fused RMSNorm, fused SwiGLU and the fused
 * reversible residual updates (midpoint and Hamiltonian-Euler).
 *
 * Conventions shared by every entry point
 *   - Pointers are device pointers (HIP global memory).  Tensors are dense and
 *     row-major; a row is `width` (or `ld`) elements long.
 *   - `stream` is a hipStream_t passed as void* (NULL = the legacy default
 *     stream).  Every call is asynchronous: it enqueues kernels on `stream`,
 *     never synchronises the host and never allocates memory.
 *   - The return value is an rv_status: 0 on success; otherwise the launch did
 *     not happen (argument errors) or HIP reported an error at launch time.
 *     rv_status_string() names a code.
 *   - Results do not depend on the launch shape or on the number of compute
 *     units: every reduction has a fixed order, there are no float atomics, and
 *     two calls on identical inputs give bit-identical outputs.
 *   - Floating-point expressions keep the operation order of the reference's
 *     kernels and are compiled without FMA contraction.
 *
 * Reference interfaces each entry point replaces are cited as
 * path:line under the LokeshJatangi/Reversability source tree.
 */
#ifndef REVERSIBILITY_HIP_H
#define REVERSIBILITY_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum rv_status {
  RV_OK = 0,
  RV_ERR_NULL_POINTER = 1,   /* a required pointer is NULL                     */
  RV_ERR_BAD_SIZE = 2,       /* negative/zero size, ld < width, ...            */
  RV_ERR_UNSUPPORTED = 3,    /* dtype or width outside what the kernels cover  */
  RV_ERR_WORKSPACE = 4,      /* workspace missing or smaller than required     */
  RV_ERR_HIP = 5             /* HIP runtime reported an error at launch        */
} rv_status;

typedef enum rv_dtype {
  RV_F32 = 0,
  RV_F16 = 1,
  RV_BF16 = 2,
  RV_F64 = 3
} rv_dtype;

/* Human-readable name of a status code (static storage). */
const char* rv_status_string(int status);

/* Last HIP error text seen by this thread's most recent failing call. */
const char* rv_last_error(void);

/* ABI version of this header: bumped when a signature changes. */
int rv_abi_version(void);

/* ------------------------------------------------------------------------
 * RMSNorm over the last dimension, FP32.
 *   y[r, c]  = (x[r, c] * rstd[r]) * w[c]
 *   rstd[r]  = rsqrt(sum_c x[r, c]^2 / width + eps)
 * Replaces _rms_forward + FusedRMSNorm.forward
 *   (src/reversibility/kernels_v3.py:9-16, 51-62).
 * width <= 4096.
 */
int rv_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd,
                   int64_t rows, int64_t width, float eps, void* stream);

/* Bytes of scratch rv_rmsnorm_bwd needs for (rows, width) on the current
 * device.  Returns a negative rv_status on bad sizes. */
int64_t rv_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t width);

/* RMSNorm backward, FP32, single pass over x and dy:
 *   g        = dy * w
 *   dx[r, :] = (g - x * ((sum_c g*x) / width * rstd * rstd)) * rstd
 *   dw[c]    = sum_r dy[r, c] * (x[r, c] * rstd[r])
 * dw is reduced from per-block partial sums in a fixed order (second, small
 * kernel).  `workspace` is device memory of at least
 * rv_rmsnorm_bwd_workspace_bytes(rows, width) bytes; its contents on entry
 * do not matter.
 * Replaces _rms_dx + _rms_dw_partials + _rms_dw_reduce + FusedRMSNorm.backward
 *   (src/reversibility/kernels_v3.py:19-48, 64-74).
 */
int rv_rmsnorm_bwd(const float* x, const float* w, const float* dy,
                   const float* rstd, float* dx, float* dw, void* workspace,
                   int64_t workspace_bytes, int64_t rows, int64_t width,
                   void* stream);

/* rv_rmsnorm_bwd without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference: it is
 * rv_rmsnorm_bwd's computation (the same kernels, bit-identical dx and dw)
 * with the dweight partial sums kept in a static device array of 4 MiB
 * (256 x 4096 fp32) that each GPU holds from the first call on that device
 * until the process ends.  The call allocates nothing (no hipMalloc / hipFree,
 * no library allocation); its first call on a device looks up the array's
 * address there (hipGetSymbolAddress, no stream work: that first call may be
 * made under graph capture).  width <= 4096 (RV_ERR_UNSUPPORTED above); the partial rows
 * (rv_rmsnorm_bwd_workspace_bytes) must fit the 4 MiB array -- for width <=
 * 256 one partial row per ceil(rows / 256) rows (16 .. 128), so rows <=
 * 524288 at width 256;
 * above 256 any rows (256 partial rows) -- (RV_ERR_WORKSPACE otherwise); and
 * the stream (if not null) must belong to the current device
 * (RV_ERR_UNSUPPORTED otherwise).  All calls on one GPU
 * share the array: calls that overlap on one GPU (concurrent streams,
 * threads) race and must be ordered by the caller. */
int rv_rmsnorm_bwd_noalloc(const float* x, const float* w, const float* dy,
                           const float* rstd, float* dx, float* dw,
                           int64_t rows, int64_t width, void* stream);

/* ------------------------------------------------------------------------
 * SwiGLU over a packed up-projection u[rows, ld_u]: gate = u[:, 0:width],
 * value = u[:, width:2*width].  dtype is RV_F16 or RV_F32.
 *   o[r, c] = round_dtype(silu(gate)) * value        (o is [rows, width])
 * silu is computed in FP32 and rounded to the I/O dtype before the multiply.
 * Replaces _swiglu_forward + FusedSwiGLU.forward
 *   (src/reversibility/kernels.py:88-95, 113-122).
 * ld_u >= 2*width.
 */
int rv_swiglu_fwd(const void* u, int64_t ld_u, void* o, int64_t rows,
                  int64_t width, int dtype, void* stream);

/* SwiGLU backward into the packed gradient du[rows, ld_u]:
 *   s          = sigmoid(gate)
 *   du[:, gate]  = round(dy * value) * (s * (1 + gate * (1 - s)))
 *   du[:, value] = dy * round(gate * s)
 * Columns of du beyond 2*width (if ld_u > 2*width) are left untouched.
 * Replaces _swiglu_backward + FusedSwiGLU.backward
 *   (src/reversibility/kernels.py:98-110, 124-131).
 */
int rv_swiglu_bwd(const void* u, int64_t ld_u, const void* dy, void* du,
                  int64_t rows, int64_t width, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Fused midpoint residual update (paper Eq. 2.4/2.5):
 *   f      = round_T(a + m)                  (attention + MLP terms)
 *   out[i] = p[i] + sign * S(round_T(f * scale))
 * with p/out in state dtype S (RV_F32 or RV_F64) and a, m in force dtype T
 * (RV_F16, RV_BF16, RV_F32 or RV_F64, T no wider than S).  scale is 2*h.
 * sign = +1 is forward_pair's p + 2h f(q); sign = -1 is inverse_pair's
 * q - 2h f(p).  out may alias p.
 * Replaces the eager residual arithmetic of midpoint_force/forward_pair/
 * inverse_pair (src/reversibility/reversible.py:16-18, 21-24, 28-30).
 */
int rv_midpoint_update(const void* p, const void* a, const void* m, void* out,
                       double scale, int sign, int64_t n, int state_dtype,
                       int force_dtype, void* stream);

/* Gradient of rv_midpoint_update with respect to a and m (both equal):
 *   da[i] = round_T(round_T(dout[i]) * scale) * sign
 * dout is in the state dtype, da in the force dtype.  (The gradient with
 * respect to p is dout itself.)  Matches autograd through the eager
 * expression, including the cast of the FP32 gradient to the force dtype.
 */
int rv_midpoint_update_bwd(const void* dout, void* da, double scale, int sign,
                           int64_t n, int state_dtype, int force_dtype,
                           void* stream);

/* Hamiltonian-Euler residual update (paper Eq. 2.8/2.9):
 *   out[i] = x[i] + sign * S(f[i])
 * sign = +1: q + A(p), p + M(q');  sign = -1: p - M(q), q - A(p0).
 * Replaces the eager adds of forward_pair/inverse_pair, Euler branch
 *   (src/reversibility/reversible.py:24-25, 31-32).
 */
int rv_residual_axpy(const void* x, const void* f, void* out, int sign,
                     int64_t n, int state_dtype, int force_dtype,
                     void* stream);

/* rv_rmsnorm_fwd with y written as fp16 (rounded to nearest even): the
 * value fp16 autocast feeds the GEMM that consumes y (FusedRMSNorm's output
 * under torch.autocast(float16), src/reversibility/kernels_v3.py:51-83).
 * width % 4 == 0; x, w 16-byte aligned, y 8-byte aligned. */
int rv_rmsnorm_fwd_f16(const float* x, const float* w, void* y, float* rstd,
                       int64_t rows, int64_t width, float eps, void* stream);

/* rv_rmsnorm_bwd with dy given as fp16 (the consuming GEMM's input gradient,
 * which autocast widens to fp32 without change); same results bit for bit.
 * width % 4 == 0; x, w, dx 16-byte aligned, dy 8-byte aligned. */
int rv_rmsnorm_bwd_f16(const float* x, const float* w, const void* dy,
                       const float* rstd, float* dx, float* dw, void* workspace,
                       int64_t workspace_bytes, int64_t rows, int64_t width,
                       void* stream);

/* The fused residual add + RMSNorm with the fp16 output: h = x + f (fp32),
 * y = fp16(norm(h)), rstd; the midpoint force's x + A(x) and the Euler step's
 * q + A(p) feeding M's norm (src/reversibility/reversible.py:16-25).  f fp32
 * (RV_F32) or fp16 (RV_F16); vector path only (width % 4 == 0, aligned). */
int rv_add_rmsnorm_fwd_f16(const float* x, const void* f, int force_dtype, const float* w,
                           float* h, void* y, float* rstd, int64_t rows, int64_t width,
                           float eps, void* stream);

/* rv_rmsnorm_bwd with dy fp32 (RV_F32) or fp16 (RV_F16), plus: dx += dh when
 * dh is given (the gradient of the normalized input's other uses, added as
 * autograd's accumulation would), and dx16 = fp16(dx) when dx16 is given
 * (the gradient of an fp16 force term of the add).  Same workspace as
 * rv_rmsnorm_bwd; with dh or dx16 only the vector path (else
 * RV_ERR_UNSUPPORTED). */
int rv_rmsnorm_bwd_acc(const float* x, const float* w, const void* dy, int dy_dtype,
                       const float* rstd, const float* dh, float* dx, void* dx16, float* dw,
                       void* workspace, int64_t workspace_bytes, int64_t rows, int64_t width,
                       void* stream);

/* rv_rmsnorm_bwd_acc for an input that also passes through unchanged to
 * another use (the split midpoint's q, an output of the rebuilt step as well
 * as the residual input of the add): dx16 = fp16(norm backward) (the force
 * term's gradient) and dx = norm backward + dpass (the input's total, the sum
 * autograd would form).  Requires dx16 and no dh. */
int rv_rmsnorm_bwd_acc_pass(const float* x, const float* w, const void* dy, int dy_dtype,
                            const float* rstd, const float* dh, const float* dpass, float* dx,
                            void* dx16, float* dw, void* workspace, int64_t workspace_bytes,
                            int64_t rows, int64_t width, void* stream);

/* The residual update's inverse fused into the norm that reads its result
 * (the Euler inversion, reversible.py:28-32 with kernels_v3.py:9-16):
 * d = x - f (f of dtype force_dtype: RV_F32 or RV_F16) and, with readd == 0,
 * y = fp16(RMSNorm(d)), rstd; with readd != 0 also h = d + f and
 * y = fp16(RMSNorm(h)) (the rebuilt step's sum).  The same values as
 * rv_residual_axpy(x, f, -1) followed by rv_rmsnorm_fwd_f16 (or
 * rv_add_rmsnorm_fwd_f16 of d and f), in one pass.  Vector path only:
 * width % 4 == 0, x, w, d, h 16-byte aligned, y 8-byte aligned. */
int rv_sub_rmsnorm_fwd_f16(const float* x, const void* f, int force_dtype, int readd,
                           const float* w, float* d, float* h, void* y, float* rstd,
                           int64_t rows, int64_t width, float eps, void* stream);

/* The midpoint update fused into the norm that reads its result next (the
 * next layer's attn_norm of next_q, reversible.py:21-25 / the reconstruction's
 * prev_p, reversible.py:28-32, with kernels_v3.py:9-16): out = p +/- fp16(fp16(a
 * + m) * scale) (sign +1 / -1; a, m fp16, the eager rounding points of
 * rv_midpoint_update) and y = fp16(RMSNorm(out)), rstd -- the same values as
 * rv_midpoint_update followed by rv_rmsnorm_fwd_f16, in one pass.  Vector
 * path only: width % 4 == 0, p, w, out 16-byte aligned, a, m, y 8-byte
 * aligned; force_dtype RV_F16. */
int rv_midpoint_rmsnorm_fwd_f16(const float* p, const void* a, const void* m, int force_dtype,
                                double scale, int sign, const float* w, float* out, void* y,
                                float* rstd, int64_t rows, int64_t width, float eps,
                                void* stream);

/* Fused residual add + RMSNorm (the x + A(x) -> mlp_norm step of
 * midpoint_force and the q' = q + A(p) -> mlp_norm step of Euler):
 *   h[r, :] = x[r, :] + S(f[r, :])             (written to h)
 *   y, rstd = RMSNorm(h) as in rv_rmsnorm_fwd
 * x, h, y: FP32; f: RV_F16, RV_BF16 or RV_F32.  h may alias x.
 * Replaces the eager `x + attention` / `q + block.attn(...)` followed by
 * block.mlp_norm (src/reversibility/reversible.py:17-18, 24-25;
 * src/reversibility/kernels_v3.py:9-16).
 */
int rv_add_rmsnorm_fwd(const float* x, const void* f, int force_dtype,
                       const float* w, float* h, float* y, float* rstd,
                       int64_t rows, int64_t width, float eps, void* stream);

/* ------------------------------------------------------------------------
 * MLP projections on MFMA (v_mfma_f32_32x32x16_f16), fp16 operands with fp32
 * accumulation, for one token tile of the SwiGLU MLP under fp16 autocast.
 * Weights are fp16 copies of the fp32 masters (W_up [2f, d] = [gate; value]
 * rows, W_down [d, f]) made by rv_cast_f32_f16, which is the cast autocast's
 * F.linear applies; activations are fp16.  d and f must be multiples of 128,
 * rows is free, row strides are multiples of 8 elements, pointers 16-byte
 * aligned.  Together these replace the F.linear / FusedSwiGLU / autograd.grad
 * calls of mlp_value and TiledMLP (src/reversibility/optimized_v3.py:10-18,
 * 29-63; src/reversibility/model.py:54-56).
 */

/* dst[i] = fp16(src[i]) (round to nearest even), i < n: autocast's cast of an
 * fp32 weight or activation for an fp16 F.linear
 * (src/reversibility/optimized_v3.py:15-17 under torch.autocast). */
int rv_cast_f32_f16(const float* src, void* dst, int64_t n, void* stream);

/* The same cast for count <= rv_cast_f32_f16_max_tensors() tensors in one
 * launch (dst[i][j] = fp16(src[i][j]), j < numel[i]; 16-byte aligned
 * pointers): all of a step's weight casts at once instead of one launch per
 * weight and evaluation. */
int rv_cast_f32_f16_max_tensors(void);
int rv_cast_f32_f16_multi(int count, const float* const* src, void* const* dst,
                          const int64_t* numel, void* stream);

/* o[rows, f] = fp16(silu(fp16(u_g))) * fp16(u_v), u = x W_up^T; x fp16 with
 * row stride ldx, w_up fp16 [2f, d].  If u is not NULL the fp16
 * pre-activation u[rows, 2f] = [u_g | u_v] is written too. */
int rv_mlp_up_swiglu(const void* x, int64_t ldx, const void* w_up, int64_t rows,
                     int64_t d, int64_t f, void* o, void* u, void* stream);

/* y[rows, d] = fp16(o W_down^T), o fp16 [rows, f], w_down fp16 [d, f]. */
int rv_mlp_down(const void* o, const void* w_down, int64_t rows, int64_t d,
                int64_t f, void* y, void* stream);

/* du[rows, 2f] = SwiGLU backward of u at d_o = fp16(dy W_down), with the
 * rounding points of rv_swiglu_bwd; dy fp16 [rows, d], u fp16 [rows, 2f],
 * w_down fp16 [d, f]. */
int rv_mlp_dgate(const void* dy, const void* w_down, const void* u,
                 int64_t rows, int64_t d, int64_t f, void* du, void* stream);

/* dx[rows, d] = fp32(fp16(du W_up)), du fp16 [rows, 2f], w_up fp16 [2f, d]. */
int rv_mlp_dx(const void* du, const void* w_up, int64_t rows, int64_t d,
              int64_t f, float* dx, void* stream);

/* Scratch bytes rv_mlp_wgrad needs (split-K partial sums; may be 0). */
int64_t rv_mlp_wgrad_workspace_bytes(int64_t rows, int64_t d, int64_t f);

/* Weight gradients of one tile, reduced over its tokens in a fixed order:
 *   ddown[d, f]  (+)= fp32(fp16(dy^T o))
 *   dup[2f, d]   (+)= fp32(fp16(du^T x))
 * dy, o, du, x fp16 (x with row stride ldx); accumulate = 0 overwrites,
 * 1 adds (the per-tile fp32 sum of TiledMLP). */
int rv_mlp_wgrad(const void* dy, const void* o, const void* du, const void* x,
                 int64_t ldx, int64_t rows, int64_t d, int64_t f,
                 float* ddown, float* dup, int accumulate, void* workspace,
                 int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Bias-free linear layers under fp16 autocast on the same MFMA kernels: the
 * attention's qkv and output projections (src/reversibility/model.py:26-45,
 * nn.Linear under torch.autocast, as called from midpoint_force /
 * forward_pair, src/reversibility/reversible.py:16-25).  x and dy fp16,
 * w fp16 [out, in] (cast once per call with rv_cast_f32_f16); in and out
 * multiples of 128.
 */

/* y[rows, out] = fp16(x W^T), x with row stride ldx. */
int rv_linear_fwd(const void* x, int64_t ldx, const void* w, int64_t rows,
                  int64_t in, int64_t out, void* y, void* stream);

/* dx[rows, in] = fp16(dy W), widened to fp32 when dx_dtype == RV_F32 (the
 * gradient autocast returns for an fp32 input). */
int rv_linear_dx(const void* dy, const void* w, int64_t rows, int64_t in,
                 int64_t out, void* dx, int dx_dtype, void* stream);

/* Scratch bytes rv_linear_dw needs (split-K partial sums; may be 0). */
int64_t rv_linear_dw_workspace_bytes(int64_t rows, int64_t in, int64_t out);

/* dw[out, in] (+)= fp32(fp16(dy^T x)), reduced over the rows in a fixed order
 * (the fp32 master-weight gradient autocast produces). */
int rv_linear_dw(const void* dy, const void* x, int64_t ldx, int64_t rows,
                 int64_t in, int64_t out, float* dw, int accumulate,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* Tile-shape control of the activation GEMMs above (rv_mlp_up_swiglu,
 * rv_mlp_down, rv_mlp_dgate, rv_mlp_dx, rv_linear_fwd, rv_linear_dx).  No
 * counterpart in the reference (cuBLAS picks its own kernels): a diagnostic
 * and test hook.  The shape never changes a result bit.  By default each
 * (epilogue, layouts, m, n, k) takes the fastest shape measured on its first
 * call; rv_gemm_force_shape(i) makes every later call use shape i
 * (0 <= i < rv_gemm_num_shapes(); RV_ERR_UNSUPPORTED from a call whose width
 * the shape does not divide), -1 restores the default.  Process-wide. */
int rv_gemm_num_shapes(void);
int rv_gemm_force_shape(int shape);

/* ------------------------------------------------------------------------
 * AdamW (decoupled weight decay) over fp32 parameters, torch.optim.AdamW's
 * arithmetic and operation order, as the training step drives it through
 * torch.amp.GradScaler (scripts/benchmark_optimized.py:38-40, 66-80;
 * scripts/train_baseline.py:270-284).  The step count is a device fp32 per
 * parameter group.
 */

/* Largest tensor count one rv_adamw_step call accepts. */
int rv_adamw_max_tensors(void);

/* *step += 1 unless found_inf is given and *found_inf != 0. */
int rv_adamw_advance(float* step, const float* found_inf, void* stream);

/* One update of count tensors (arrays of device pointers and sizes in host
 * memory): p, m, v updated in place from g (times *inv_scale if given), with
 * the bias corrections of the (already advanced) *step; nothing changes when
 * found_inf is given and *found_inf != 0. */
int rv_adamw_step(int count, float* const* params, const float* const* grads,
                  float* const* exp_avg, float* const* exp_avg_sq,
                  const int64_t* numel, double lr, double beta1, double beta2,
                  double eps, double weight_decay, const float* step,
                  const float* found_inf, const float* inv_scale, void* stream);

/* rv_adamw_step with clip_grad_norm_'s multiply as well: g times *inv_scale
 * (if given), rounded, times *clip_coef (if given), rounded -- the values
 * GradScaler.unscale_ and clip_grad_norm_ would have written into the
 * gradients -- so those two passes need not write them. */
int rv_adamw_step_clipped(int count, float* const* params, const float* const* grads,
                          float* const* exp_avg, float* const* exp_avg_sq,
                          const int64_t* numel, double lr, double beta1, double beta2,
                          double eps, double weight_decay, const float* step,
                          const float* found_inf, const float* inv_scale,
                          const float* clip_coef, void* stream);

/* GradScaler.unscale_ followed by torch.nn.utils.clip_grad_norm_(params,
 * max_norm) (norm type 2; scripts/train_baseline.py:278-280) without writing
 * the gradients: rv_grad_sq_partials stores, for each 16384-element chunk of
 * each of count <= rv_adamw_max_tensors() gradients, the fp32 sum of squares
 * of g * *inv_scale (inv_scale nullable) and a non-finite flag at index
 * first + chunk of partials / flags (rv_grad_chunks(numel, count) chunks; a
 * negative return is -status); rv_grad_clip_coef reduces n partials in a
 * fixed order to total_norm = sqrt(sum), clip_coef = min(max_norm /
 * (total_norm + 1e-6), 1) and found_inf = 1 if any chunk was non-finite
 * (0 otherwise), all device fp32 scalars for rv_adamw_step_clipped. */
int rv_grad_chunks(const int64_t* numel, int count);
int rv_grad_sq_partials(int count, const float* const* grads, const int64_t* numel,
                        const float* inv_scale, float* partials, float* flags, int first,
                        void* stream);
int rv_grad_clip_coef(const float* partials, const float* flags, int n, double max_norm,
                      float* total_norm, float* clip_coef, float* found_inf, void* stream);

/* ------------------------------------------------------------------------
 * Cross-entropy over vocabulary rows (the tied LM head's loss).
 * logits [rows, ld] fp16 (RV_F16) or fp32 (RV_F32), first cols columns used;
 * labels int64 [rows]; rows whose label equals ignore_index contribute 0.
 * Replace TiledCrossEntropy's _ce_partials / _ce_rows / _ce_grad launches
 * (src/reversibility/kernels.py:14-77).
 */

/* row_max = max_j x_j, row_lse = log(sum_j exp(x_j - row_max)) and
 * loss = -round_T((x_t - row_max) - row_lse), all fp32 [rows]; a label
 * outside [0, cols) other than ignore_index gives a NaN loss. */
int rv_ce_fwd(const void* logits, int dtype, int64_t ld, const int64_t* labels,
              int64_t rows, int64_t cols, int64_t ignore_index, float* row_max,
              float* row_lse, float* loss, void* stream);

/* dlogits (layout and dtype of logits) = gradient of sum(loss) times *grad
 * (a device fp32 scalar): round_T([j == t] n - exp(round_T((x_j - row_max) -
 * row_lse)) n), n = round_T(-*grad); zero rows for ignore_index.  logits and
 * dlogits must share their address modulo 16. */
int rv_ce_bwd(const void* logits, int dtype, int64_t ld, const int64_t* labels,
              const float* row_max, const float* row_lse, const float* grad,
              int64_t rows, int64_t cols, int64_t ignore_index, void* dlogits,
              void* stream);

/* rv_ce_fwd followed by rv_ce_bwd in one pass over the logits (each row is
 * read once and kept in registers), with the same results bit for bit; for
 * callers that know the upstream gradient *grad before the forward (the tied
 * head's chunked trainer, src/reversibility/optimized_v3.py:168-186, which
 * runs the loss forward and backward of one chunk back to back).  fp16 only and
 * cols <= 65536 (else RV_ERR_UNSUPPORTED: use the two calls).  dlogits may
 * be logits itself (in place). */
int rv_ce_fused(const void* logits, int dtype, int64_t ld, const int64_t* labels,
                int64_t rows, int64_t cols, int64_t ignore_index, const float* grad,
                float* row_max, float* row_lse, float* loss, void* dlogits,
                void* stream);

/* ------------------------------------------------------------------------
 * Causal self-attention (F.scaled_dot_product_attention(q, k, v,
 * is_causal=True), default scale 1/sqrt(head_dim), src/reversibility/
 * model.py:40-45) on the packed projection.  qkv fp16 [batch, seq, 3, heads,
 * head_dim] as the qkv GEMM writes it; out / dout fp16 [batch, seq, heads,
 * head_dim]; lse fp32 [batch * heads, seq] (base-2 log-sum-exp of the scaled
 * scores); head_dim 32, 64 or 128; fp16 pointers 16-byte aligned.
 */

/* out = softmax(q k^T / sqrt(head_dim), causal) v; lse for the backward. */
int rv_attn_fwd(const void* qkv, int64_t batch, int64_t seq, int64_t heads,
                int64_t head_dim, void* out, float* lse, void* stream);

/* Workspace bytes of rv_attn_bwd (negative: -error). */
int64_t rv_attn_bwd_workspace_bytes(int64_t batch, int64_t seq, int64_t heads);

/* dqkv (fp16, qkv's layout) = gradient of out with respect to qkv, given
 * dout and the forward's out and lse.  Deterministic. */
int rv_attn_bwd(const void* qkv, const void* out, const void* dout, const float* lse,
                int64_t batch, int64_t seq, int64_t heads, int64_t head_dim,
                void* dqkv, void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Token pipeline and token + position embedding (the steps in front of the
 * reversible stack).  Tables and activations fp32, d a multiple of 4, fp32
 * pointers 16-byte aligned.
 */

/* batch_at (scripts/train_baseline.py:50-63) on a device window of count + 1
 * uint16 tokens: x[i] = window[i], y[i] = window[i + 1] for i < count, then
 * x = 0, y = -100 up to ceil(count / seq_len) * seq_len entries (int64). */
int rv_batch_from_tokens(const uint16_t* window, int64_t count, int64_t seq_len,
                         int64_t* x, int64_t* y, void* stream);

/* out[b, t] = tok[ids[b, t]] + pos[t] (src/reversibility/reversible.py:105-106,
 * the boundary p = q = embedding; model.py's token and position
 * nn.Embedding).  An id outside [0, vocab) gives a NaN row. */
int rv_embed_fwd(const int64_t* ids, int64_t batch, int64_t seq, const float* tok,
                 int64_t vocab, const float* pos, int64_t max_seq, int64_t d,
                 float* out, void* stream);

/* Workspace bytes rv_embed_bwd needs for this many tokens (negative: -error). */
int64_t rv_embed_bwd_workspace_bytes(int64_t tokens, int64_t vocab, int64_t d);

/* The embedding's backward, deterministic: dtok[v] (+)= sum of dout rows
 * whose id is v (nn.Embedding's weight gradient; rows of untouched ids are
 * zeroed unless accumulating, ids outside [0, vocab) get nothing) and
 * dpos[t] (+)= sum_b dout[b, t] (the position embedding's gradient through
 * the broadcast add; rows seq <= t < max_seq zeroed unless accumulating).
 * Either output may be NULL. */
int rv_embed_bwd(const int64_t* ids, int64_t batch, int64_t seq, const float* dout,
                 int64_t vocab, int64_t max_seq, int64_t d, float* dtok,
                 int tok_accumulate, float* dpos, int pos_accumulate,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Measurement only (no counterpart in the reference; no hot-path result
 * depends on them): the streaming floor a bandwidth-bound kernel is judged
 * against.
 */

/* Read nin (1..3) arrays and write nout (1..2) arrays of `bytes` bytes each
 * (a multiple of 16; 16-byte aligned device pointers; `in` and `out` are host
 * arrays of device pointers), 16 bytes per access, `vec` (1, 2, 4 or 8)
 * vectors per array and thread, every load issued before the first wait;
 * hints bit 0 = non-temporal loads, bit 1 = non-temporal stores.  Each output
 * is the xor of the inputs (output k with k xored into its first word). */
int rv_stream_floor(const void* const* in, int nin, void* const* out, int nout, int64_t bytes,
                    int vec, int hints, void* stream);

/* An empty kernel of `blocks` workgroups: the cost of one more launch. */
int rv_empty_kernel(int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* REVERSIBILITY_HIP_H */
