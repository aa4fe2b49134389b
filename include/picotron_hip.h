/*
 * picotron_hip.h -- C ABI of libpicotron_hip.so, the gfx950 (MI355X) kernels behind
 * picotron's optional fused-kernel surface (picotron.nn.triton_kernels).
 *
 * Every entry point is extern "C", takes plain device pointers, element counts and
 * strides, and an explicit HIP stream (passed as void*; NULL means the default stream).
 * The library never allocates or frees device memory: the caller owns every buffer,
 * including workspaces, whose sizes the *_workspace_bytes() queries return.
 *
 * Return value: PT_OK (0) on success, otherwise a PT_E* code; pt_last_error() then
 * returns a message for the calling thread.  Validation happens on the host before
 * any launch, so a nonzero return means nothing was enqueued.  Asynchronous device
 * faults are not reported here (as with any HIP launch).
 *
 * Strides and counts are in ELEMENTS, not bytes.  The innermost (hidden / head_dim /
 * vocab) dimension must be contiguous (stride 1).
 *
 * Reference interfaces (AndyMLAndAI/picotron) that these entry points replace are
 * cited as path:line relative to the reference repository root.
 */
#ifndef PICOTRON_HIP_H
#define PICOTRON_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PT_ABI_VERSION 4

/* element type codes (storage types; arithmetic is always fp32) */
#define PT_FLOAT32 0
#define PT_FLOAT16 1
#define PT_BFLOAT16 2

/* return codes */
#define PT_OK 0
#define PT_EINVAL 1        /* bad argument: null pointer, shape, stride, alignment */
#define PT_EUNSUPPORTED 2  /* valid request the library does not handle (dtype, size) */
#define PT_ELAUNCH 3       /* hipGetLastError() reported a launch failure */
#define PT_EDEVICE 4       /* no usable gfx950 device / HIP runtime error */

/* ABI version of the loaded library; must equal PT_ABI_VERSION. */
int pt_abi_version(void);

/* Message for the last nonzero return on the calling thread ("" if none). */
const char* pt_last_error(void);

/* 1 if `device` is a gfx950 GPU this library was built for, 0 otherwise.
 * Replaces the capability gate of src/picotron/utils/hardware.py:93-108
 * (detect_triton_support: capability >= 7) and the per-op checks at
 * src/picotron/nn/triton_kernels/rmsnorm.py:142-145, swiglu.py:89-92. */
int pt_device_supported(int device);

/* ---------------------------------------------------------------- RMSNorm
 * y[r, :] = (x[r, :] * rstd[r]) * w,   rstd[r] = 1 / sqrt(mean(x[r, :]^2) + eps)
 * computed in fp32, stored in x's type; rstd is written in fp32 for the backward.
 * Replaces _rmsnorm_kernel + _run_triton_forward (src/picotron/nn/triton_kernels/
 * rmsnorm.py:25-46, 63-84) and _inverse_rms (rmsnorm.py:49-53), which the reference
 * runs as a separate full pass on every forward (rmsnorm.py:103).
 * x_dtype: type of x and y.  w_dtype: type of weight (any of the three). */
int pt_rmsnorm_fwd(const void* x, int64_t x_row_stride, const void* weight, void* y,
                   int64_t y_row_stride, float* rstd, int64_t rows, int64_t cols, float eps,
                   int x_dtype, int w_dtype, void* stream);

/* Bytes of fp32 workspace pt_rmsnorm_bwd needs for the weight-gradient partials. */
size_t pt_rmsnorm_bwd_workspace_bytes(int64_t rows, int64_t cols, int x_dtype);

/* dx = rstd * (dy*w - x * rstd^2 * mean(dy*w*x)),  dweight = sum_rows(dy * x * rstd)
 * Replaces the PyTorch-eager backward of _RMSNormAutogradFunction
 * (src/picotron/nn/triton_kernels/rmsnorm.py:110-134).  dx may be NULL (no input grad);
 * dweight may be NULL (no weight grad; workspace then unused).  dy has x's type, dx is
 * written in x's type and dweight in w's type.  The weight reduction is deterministic:
 * per-block fp32 partials in `workspace`, then a fixed-order column sum. */
int pt_rmsnorm_bwd(const void* dy, int64_t dy_row_stride, const void* x, int64_t x_row_stride,
                   const void* weight, const float* rstd, void* dx, int64_t dx_row_stride,
                   void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
                   int64_t cols, int x_dtype, int w_dtype, void* stream);

/* pt_rmsnorm_bwd without a workspace argument, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  No counterpart in the reference.  The weight-gradient partials go to a
 * static device array of the library (16 MiB, one per device, held until the process
 * ends); the call allocates and frees nothing.  Same arguments and results as
 * pt_rmsnorm_bwd (bitwise: same kernels and grid).  Returns PT_EUNSUPPORTED when the
 * partials, pt_rmsnorm_bwd_workspace_bytes(rows, cols, x_dtype), exceed 16 MiB (e.g. more
 * than 8192 columns at 16384 rows).  Calls that overlap on one device share the array and
 * race: issue them on one stream, or serialise them.  The first call on a device looks up
 * the array's device address and must not be made inside a graph capture (it returns
 * PT_EUNSUPPORTED there); later calls can be captured and replayed. */
int pt_rmsnorm_bwd_noalloc(const void* dy, int64_t dy_row_stride, const void* x,
                           int64_t x_row_stride, const void* weight, const float* rstd, void* dx,
                           int64_t dx_row_stride, void* dweight, int64_t rows, int64_t cols,
                           int x_dtype, int w_dtype, void* stream);

/* Residual add fused with the norm that follows it in the decoder block
 * (src/picotron/models/picotron_decoder.py:116-119: hidden = hidden + attention(...), then
 * mlp_norm(hidden)):  h = x + residual, computed in fp32 and rounded to x's type, is written,
 * and y = rmsnorm(h) as pt_rmsnorm_fwd computes it from the rounded h (rstd as there).  One
 * pass instead of an add pass plus a norm pass that re-reads h.  x, residual, h and y share
 * x_dtype; h must not be x, residual or y. */
int pt_residual_rmsnorm_fwd(const void* x, int64_t x_row_stride, const void* residual,
                            int64_t residual_row_stride, const void* weight, void* h,
                            int64_t h_row_stride, void* y, int64_t y_row_stride, float* rstd,
                            int64_t rows, int64_t cols, float eps, int x_dtype, int w_dtype,
                            void* stream);

/* Backward of the fused add + norm.  h also feeds the block's final residual add, so its
 * gradient is the norm's input gradient plus the gradient arriving from that add:
 *   dh = rmsnorm_backward(dy; h, weight, rstd) + dh_in   (fp32, rounded once)
 * which is also the gradient of both x and residual.  dh_in may be NULL (then this is
 * pt_rmsnorm_bwd with dx = dh) and dh may be the same buffer as dh_in (accumulate in place).
 * dweight and the workspace as in pt_rmsnorm_bwd. */
int pt_residual_rmsnorm_bwd(const void* dy, int64_t dy_row_stride, const void* dh_in,
                            int64_t dh_in_row_stride, const void* h, int64_t h_row_stride,
                            const void* weight, const float* rstd, void* dh, int64_t dh_row_stride,
                            void* dweight, void* workspace, size_t workspace_bytes, int64_t rows,
                            int64_t cols, int x_dtype, int w_dtype, void* stream);

/* ---------------------------------------------------------------- SwiGLU
 * out = gate * sigmoid(gate) * up over n contiguous elements (fp32 math).
 * Replaces _swiglu_kernel + _run_triton_forward (src/picotron/nn/triton_kernels/
 * swiglu.py:26-53). */
int pt_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dtype,
                  void* stream);

/* s = sigmoid(g); dgate = dout * up * s * (1 + g * (1 - s)); dup = dout * g * s.
 * Replaces the eager backward of _SwiGLUAutogradFunction (swiglu.py:71-81), computed
 * in fp32 instead of the input type.  dgate or dup may be NULL to skip that output. */
int pt_swiglu_bwd(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                  int64_t n, int dtype, void* stream);

/* ---------------------------------------------------------------- RoPE
 * Rotary embedding of up to two tensors (query and key) in one launch.  Each tensor is a
 * logical (batch, heads, seq, head_dim) view described by
 *   desc[9] = {batch, heads, seq, x_stride_batch, x_stride_head, x_stride_seq,
 *              y_stride_batch, y_stride_head, y_stride_seq}
 * with head_dim contiguous.  Position of sequence index s is table row s; cos_table and
 * sin_table are fp32 [table_rows, head_dim/2] (table_rows >= seq).
 * layout 0 = interleaved pairs (2i, 2i+1), as in src/picotron/nn/rope.py:35-51 and the
 *            Triton kernel src/picotron/nn/triton_kernels/rope.py:25-49;
 * layout 1 = rotate-half pairs (i, i + head_dim/2).
 * inverse = 1 rotates by -angle (the backward of the forward rotation).
 * x1/y1/desc1 may be NULL for a single tensor.  y may alias x (in place).
 * Replaces triton_apply_rotary_embedding (src/picotron/nn/triton_kernels/rope.py:52-91)
 * and, through autograd, the eager apply_rotary_embedding backward. */
int pt_rope(const void* x0, void* y0, const int64_t* desc0, const void* x1, void* y1,
            const int64_t* desc1, int64_t head_dim, const float* cos_table,
            const float* sin_table, int64_t table_rows, int layout, int inverse, int dtype,
            void* stream);

/* ---------------------------------------------------------------- Cross-entropy
 * Mean cross-entropy over rows whose target != ignore_index, fused with its gradient.
 * Row (o, i), o < outer, i < inner, starts at logits + o*outer_stride + i*inner_stride
 * and holds `vocab` contiguous logits; its target is
 * targets[o*t_outer_stride + i*t_inner_stride] (int64).  A 2-D (N, V) input is
 * outer=N, inner=1; the train loop's (B, V, S-1) view of (B, S, V) logits is
 * outer=B, inner=S-1, outer_stride=S*V, inner_stride=V.
 * loss_out (fp32 scalar, device) = sum(lse - logit[target]) / n_valid.
 * If write_grad != 0, for fp32 and bf16,
 *   d loss / d logits = (softmax - onehot(target)) / n_valid   (0 for ignored rows)
 * is written in the same pass: with grad == NULL IN PLACE over the logits; otherwise into
 * the gradient rows grad + o*grad_outer_stride + i*grad_inner_stride (vocab contiguous),
 * each starting in the same 16-byte phase as its logits row (else PT_EINVAL; the same
 * 128-byte phase also keeps the gradient's stores on whole cache lines, as the kernels split
 * rows at the logits' lines), and the logits are only read (one read of the logits and one write of the gradient either way).  fp16
 * logits are left unchanged and each row's log-sum-exp is kept in the workspace: the loss
 * scale of fp16 training arrives only with the backward, and softmax / n_valid is mostly
 * below fp16's smallest subnormal at language-model sizes, so pt_cross_entropy_scale_grad
 * (always needed for fp16) writes the gradient, scale included, rounding to fp16 once.
 * A non-ignored target outside [0, vocab) makes that row's loss NaN and sets
 * *(int32*)status bit 0; status is part of the workspace (see below).
 * Replaces CrossEntropyWithFallback / triton_cross_entropy
 * (src/picotron/nn/triton_kernels/cross_entropy.py:48-109) and the F.cross_entropy
 * fwd+bwd they fall back to. */
size_t pt_cross_entropy_workspace_bytes(int64_t rows);
int pt_cross_entropy(void* logits, int64_t outer, int64_t inner, int64_t outer_stride,
                     int64_t inner_stride, int64_t vocab, const int64_t* targets,
                     int64_t t_outer_stride, int64_t t_inner_stride, int64_t ignore_index,
                     float* loss_out, int write_grad, void* grad, int64_t grad_outer_stride,
                     int64_t grad_inner_stride, void* workspace, size_t workspace_bytes,
                     int dtype, void* stream);

/* Device address of the int32 status word inside a cross-entropy workspace. */
int32_t* pt_cross_entropy_status(void* workspace);

/* The backward of the fused loss.  `dlogits` (strides outer_stride, inner_stride) are the
 * gradient rows pt_cross_entropy wrote (the logits themselves when it worked in place; same
 * targets): multiplied in place by the fp32 scalar at *grad_output (device memory), all work
 * skipped when it equals 1.0 exactly; rows whose target is ignore_index stay zero.  For fp16
 * the gradient is written here: each element of the untouched logits, at `logits` (strides
 * logits_outer_stride, logits_inner_stride; NULL: dlogits, in place, the ABI-2 behaviour),
 * gives (exp(x - lse) - onehot) * (*grad_output / n_valid) in dlogits, computed in fp32 and
 * rounded to fp16 once (always, also for a grad_output of 1), each logits row in the same
 * 16-byte phase as its gradient row; lse and n_valid are read from `workspace`, the forward
 * call's workspace, which must then be non-NULL (fp32 and bf16 ignore `logits` and it). */
int pt_cross_entropy_scale_grad(void* dlogits, int64_t outer, int64_t inner,
                                int64_t outer_stride, int64_t inner_stride, int64_t vocab,
                                const int64_t* targets, int64_t t_outer_stride,
                                int64_t t_inner_stride, int64_t ignore_index,
                                const float* grad_output, const void* logits,
                                int64_t logits_outer_stride, int64_t logits_inner_stride,
                                const void* workspace, int dtype, void* stream);

/* Next-token cross-entropy on the whole (batch, seq, vocab) logits of a language model:
 * row (b, t) with t < seq-1 has target input_ids[b*ids_batch_stride + (t+1)*ids_seq_stride];
 * the rows of the last position t = seq-1 have no target (loss 0, not counted in n_valid,
 * gradient 0).  The loss equals pt_cross_entropy on the view
 * logits[:, :-1, :].transpose(1, 2) with targets input_ids[:, 1:] -- the train loop's call
 * at src/picotron/training/train_loop.py:141-144 -- but with write_grad the gradient
 * covers the whole (batch, seq, vocab) buffer, so autograd needs no slice backward (which
 * allocates, zero-fills and copies a full-size gradient).  Row (b, t) starts at
 * logits + b*batch_stride + t*seq_stride; with grad != NULL the gradient goes to
 * grad + b*grad_batch_stride + t*grad_seq_stride instead of over the logits (same rule as
 * pt_cross_entropy).  Workspace: pt_cross_entropy_workspace_bytes(batch * seq). */
int pt_cross_entropy_shifted(void* logits, int64_t batch, int64_t seq, int64_t batch_stride,
                             int64_t seq_stride, int64_t vocab, const int64_t* input_ids,
                             int64_t ids_batch_stride, int64_t ids_seq_stride,
                             int64_t ignore_index, float* loss_out, int write_grad, void* grad,
                             int64_t grad_batch_stride, int64_t grad_seq_stride,
                             void* workspace, size_t workspace_bytes, int dtype, void* stream);

/* pt_cross_entropy_scale_grad for a gradient written by pt_cross_entropy_shifted (same
 * description, same fp16 rule and workspace); the last position and ignored rows stay zero. */
int pt_cross_entropy_shifted_scale_grad(void* dlogits, int64_t batch, int64_t seq,
                                        int64_t batch_stride, int64_t seq_stride, int64_t vocab,
                                        const int64_t* input_ids, int64_t ids_batch_stride,
                                        int64_t ids_seq_stride, int64_t ignore_index,
                                        const float* grad_output, const void* logits,
                                        int64_t logits_batch_stride, int64_t logits_seq_stride,
                                        const void* workspace, int dtype, void* stream);

/* ---------------------------------------------------------------- AdamW
 * One decoupled-weight-decay Adam step over many fp32 tensors in one launch, with
 * torch.optim.AdamW's single-tensor arithmetic (amsgrad=False, maximize=False), per element:
 *   p *= 1 - lr*wd;  m = lerp(m, g, 1-beta1);  v = v*beta2 + ((1-beta2)*g)*g;
 *   p += -step_size * (m / (sqrt(v) / bias_correction2_sqrt + eps))
 * The library derives step_size = lr / (1 - beta1^step) and
 * bias_correction2_sqrt = (1 - beta2^step)^0.5 in double from the arguments (as torch does
 * in Python floats) and rounds every scalar to fp32 once.  `step` is the step number AFTER
 * the increment (1 on the first step).
 * `table` is a DEVICE array of n_tensors records of 6 int64:
 *   {param address, grad address, exp_avg address, exp_avg_sq address, numel,
 *    first block index}
 * where "first block index" is the running sum of ceil(numel / pt_adamw_block_elems())
 * over the preceding records (so record 0 has 0); total_blocks is the sum over all
 * records.  Every record must have numel >= 1 (a call with more records than blocks is
 * refused with PT_EINVAL), and total_blocks is at most 2^24.
 * Replaces triton_adamw_step / AdamWStepWithFallback
 * (src/picotron/nn/triton_kernels/adamw.py:14-47), which always raises today, and the
 * torch.optim.AdamW step it falls back to (src/picotron/training/train_loop.py:308-325). */
int64_t pt_adamw_block_elems(void);
int pt_adamw_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks, double lr,
                  double beta1, double beta2, double eps, double weight_decay, double step,
                  void* stream);

/* Gradient clipping fused into the step.  The train loop clips right before the step
 * (src/picotron/training/train_loop.py:163-168 -> _clip_gradients :338-350 ->
 * torch.nn.utils.clip_grad_norm_(params, max_norm)), a read of every gradient for the norm
 * and a read-modify-write to scale them.  Here:
 *   pt_clip_grad_norm: total_norm = ||all gradients||_2 (fp32 per-block sums of squares,
 *     added in double in a fixed order) and clip_coef = min(max_norm / (total_norm + 1e-6), 1)
 *     as torch computes it, written as fp32 scalars to device memory.  `table` has the
 *     pt_adamw_step layout; only the grad address, numel and first block index are read.
 *     Workspace: pt_clip_grad_norm_workspace_bytes(total_blocks).  With no records,
 *     total_norm = 0 and clip_coef = 1.
 *   pt_adamw_step_scaled: pt_adamw_step with every gradient multiplied by *grad_scale
 *     (device fp32, e.g. clip_coef) as it is read, g = g * scale as torch's clipping
 *     leaves it; with write_grad != 0 the scaled gradient is also stored back, so the
 *     gradients end exactly as after torch's clip_grad_norm_. */
size_t pt_clip_grad_norm_workspace_bytes(int64_t total_blocks);
int pt_clip_grad_norm(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                      double max_norm, float* total_norm_out, float* clip_coef_out,
                      void* workspace, size_t workspace_bytes, void* stream);
int pt_adamw_step_scaled(const int64_t* table, int64_t n_tensors, int64_t total_blocks, double lr,
                         double beta1, double beta2, double eps, double weight_decay, double step,
                         const float* grad_scale, int write_grad, void* stream);

/* The step of a torch.optim.AdamW(..., capturable=True), which is what the reference's
 * fallback (optimizer.step(), src/picotron/nn/triton_kernels/adamw.py:47) runs for such an
 * optimizer: each parameter's step count is an fp32 scalar in device memory, advanced by the
 * caller before the update (torch: state["step"] += 1 on the device).  `step_table` is a
 * DEVICE array of n_tensors int64 addresses, the step of each `table` record in record
 * order.  Every workgroup reads its tensor's step t and forms, in fp32,
 * step_size = lr / (1 - beta1^t) and bias_correction2_sqrt = sqrt(1 - beta2^t); the update
 * is otherwise pt_adamw_step's.  With grad_scale non-NULL the gradients are scaled (and
 * written back when write_grad != 0) as in pt_adamw_step_scaled.  No argument depends on
 * the step's value, so the launch can be captured in a HIP graph and replayed as the step
 * advances. */
int pt_adamw_step_device_step(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                              const int64_t* step_table, double lr, double beta1, double beta2,
                              double eps, double weight_decay, const float* grad_scale,
                              int write_grad, void* stream);

/* pt_adamw_step_device_step with grad_scale, guarded by the overflow flag that pt_grad_stats
 * left on the device (found_inf, int32): when it is 0 the launch is exactly
 * pt_adamw_step_device_step; when it is set, parameters and moments are left untouched and
 * every gradient is only multiplied by *inv_scale (device fp32), as
 * torch.amp.GradScaler.unscale_ leaves the gradients of a skipped step.  The caller advances
 * the device step counts by (1 - found_inf).  It replaces the host read in the train loop's
 * fp16 update (src/picotron/training/train_loop.py:155-160: GradScaler.step reads found_inf
 * on the host to skip optimizer.step()), so that the whole fp16 update -- statistics, this
 * launch, the step counts and GradScaler.update -- runs without a host read and can be
 * captured in a HIP graph.  Added in ABI version 4. */
int pt_adamw_step_device_step_guarded(const int64_t* table, int64_t n_tensors,
                                      int64_t total_blocks, const int64_t* step_table, double lr,
                                      double beta1, double beta2, double eps,
                                      double weight_decay, const float* grad_scale,
                                      int write_grad, const int32_t* found_inf,
                                      const float* inv_scale, void* stream);

/* Mixed-precision / ZeRO gradient handling before the step
 * (src/picotron/parallel/zero.py:139-163 unscale_and_check_: a finite check of every
 * gradient, one host sync per parameter, then g *= 1/scale; :165-186 clip_grad_norm_:
 * squared norm in fp32, g *= coef when coef < 1).  One read of every gradient:
 *   pt_grad_stats: total_norm = ||g * inv_scale||_2 (inv_scale: device fp32, NULL = 1),
 *     found_inf = 1 if any g is inf or NaN, and grad_scale = inv_scale * coefficient, where
 *     for max_norm >= 0 coefficient c = (1 / (total_norm + 1e-6)) * max_norm is applied as
 *     min(c, 1) (clip_mode 0: torch.nn.utils.clip_grad_norm_) or as c if c < 1 else 1
 *     (clip_mode 1: the ZeRO optimizer), and is 1 for max_norm < 0.  Outputs are device
 *     scalars; workspace pt_grad_stats_workspace_bytes(total_blocks).  The caller reads
 *     found_inf (one sync for all tensors) and either skips the step or passes grad_scale
 *     to pt_adamw_step_scaled -- unscale, clip and step in one more pass -- or to
 *     pt_grad_scale.
 *   pt_grad_scale: g *= *scale in place for every gradient of the table (no memory traffic
 *     when *scale is exactly 1).
 * Tables have the pt_adamw_step layout (only grad address, numel, first block read). */
size_t pt_grad_stats_workspace_bytes(int64_t total_blocks);
int pt_grad_stats(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                  const float* inv_scale, double max_norm, int clip_mode, float* total_norm_out,
                  float* grad_scale_out, int32_t* found_inf_out, void* workspace,
                  size_t workspace_bytes, void* stream);
int pt_grad_scale(const int64_t* table, int64_t n_tensors, int64_t total_blocks,
                  const float* scale, void* stream);

/* ---------------------------------------------------------------- Utility
 * Device-to-device copy of `bytes` (multiple of 16, 16-byte aligned pointers) with the
 * same 128-bit load/store pattern as the streaming kernels.  No reference counterpart:
 * used by the benchmark as the achievable-bandwidth line and to calibrate rocprofv3
 * FETCH_SIZE / WRITE_SIZE against a transfer of known size. */
int pt_copy(const void* src, void* dst, int64_t bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PICOTRON_HIP_H */
