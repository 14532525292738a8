/*
 * mhc_abi.h -- C ABI of the MI355X-native (gfx950 HIP) mHC hot path.
 *
 * One shared library (libmhc_hip.so) exports the functions below.  Every
 * signature uses plain device pointers, int64 sizes, dtype codes and a HIP
 * stream handle; there are no torch types.  The Python package `mhc`
 * (mhc-triton_amd/mhc/_lib.py) binds them with ctypes; a C/C++ caller can
 * link the library directly.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers to contiguous row-major tensors.
 *   - Bulk tensors carry a dtype code (MHC_DTYPE_*); per-batch weights,
 *     parameters and weight gradients are fp32.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = legacy default
 *     stream) and the call returns without synchronising.
 *   - Return value: MHC_OK (0) or an MHC_ERR_* code; mhc_last_error()
 *     returns a message for the last failure on the calling thread.
 *   - Functions taking `workspace` need at least the number of bytes the
 *     matching *_workspace_bytes() query returns, 256-byte aligned.  The
 *     library allocates no device memory itself.
 *   - Reductions are deterministic: fixed-order trees, no float atomics.
 *
 * Shapes: B batch, S sequence, D dim (per stream), 4 streams, K = 4*D,
 * R rows of the dynamic-weight projection, N 4x4 matrices.  Entry points
 * over the stream tensor require S*D <= 2^32 - 2^16 (per-batch element
 * indices are 32-bit) and return MHC_ERR_ARG otherwise; B is unbounded.
 */
#ifndef MHC_ABI_H
#define MHC_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* mhc_stream_t; /* hipStream_t */

enum {
  MHC_DTYPE_F32 = 0,
  MHC_DTYPE_BF16 = 1,
  MHC_DTYPE_F16 = 2
};

enum {
  MHC_OK = 0,
  MHC_ERR_ARG = 1,       /* bad shape, null pointer, bad iteration count */
  MHC_ERR_DTYPE = 2,     /* unsupported dtype code */
  MHC_ERR_WORKSPACE = 3, /* workspace missing, too small or misaligned */
  MHC_ERR_HIP = 4        /* a HIP runtime call failed */
};

/* Version of this ABI (bumped on any signature or semantic change). */
int mhc_abi_version(void);

/* Message for the last non-zero status returned on the calling thread. */
const char* mhc_last_error(void);

/* ------------------------------------------------------------------------
 * Sinkhorn-Knopp projection of N independent 4x4 matrices.
 * ------------------------------------------------------------------------ */

/* Replaces sinkhorn_forward (reference src/mhc/_kernels.py:597-614, kernel
 * :30-130).  out = P after `iters` rounds of P <- P/(rowsum+eps),
 * P <- P/(colsum+eps) starting from P = |M| + eps.  M and out share `dtype`. */
int mhc_sinkhorn_forward(const void* M, void* out, int64_t n_mat, int dtype,
                         int iters, float eps, mhc_stream_t stream);

/* Replaces sinkhorn_backward (reference src/mhc/_backward.py:503-530, kernel
 * :29-262).  dM = d(sum(dP * P))/dM in dtype_M, with the derivative of |M|
 * taken as sgn(M), sgn(0) = 0 (torch autograd of the pure-PyTorch path). */
int mhc_sinkhorn_backward(const void* M, int dtype_M, const void* dP, int dtype_dP,
                          void* dM, int64_t n_mat, int iters, float eps,
                          mhc_stream_t stream);

/* ------------------------------------------------------------------------
 * Stream mix (Eq. 10-11):  branch_input[b,s,:] = sum_n H_pre[b,n] H[b,s,n,:]
 *                          H_residual[b,s,n,:] = sum_m H_res[b,n,m] H[b,s,m,:]
 * ------------------------------------------------------------------------ */

/* Replaces stream_mix_forward (reference src/mhc/_kernels.py:617-652, kernel
 * :137-236).  H [B,S,4,D], H_pre [B,4] f32, H_res [B,4,4] f32 ->
 * branch_input [B,S,D], H_residual [B,S,4,D], all bulk tensors in `dtype`. */
int mhc_stream_mix_forward(const void* H, const float* H_pre, const float* H_res,
                           void* branch_input, void* H_residual,
                           int64_t B, int64_t S, int64_t D, int dtype,
                           mhc_stream_t stream);

size_t mhc_stream_mix_backward_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype);

/* Replaces stream_mix_backward (reference src/mhc/_backward.py:578-626,
 * kernel :358-496, plus its torch .sum reductions :623-624).
 *   dH[m]       = H_pre[m] d_bi + sum_n H_res[n,m] dH_residual[n]   (dtype)
 *   dH_pre[b,n] = sum_{s,d} d_bi * H[n]                              (f32)
 *   dH_res[b,n,m] = sum_{s,d} dH_residual[n] * H[m]                  (f32) */
int mhc_stream_mix_backward(const void* d_branch_input, const void* dH_residual,
                            const void* H, const float* H_pre, const float* H_res,
                            void* dH, float* dH_pre, float* dH_res,
                            int64_t B, int64_t S, int64_t D, int dtype,
                            void* workspace, size_t workspace_bytes,
                            mhc_stream_t stream);

/* ------------------------------------------------------------------------
 * Add residual (Eq. 12):  H_new[b,s,n,:] = H_residual[b,s,n,:] + H_post[b,n] bo[b,s,:]
 * ------------------------------------------------------------------------ */

/* Replaces add_residual_forward (reference src/mhc/_kernels.py:655-687,
 * kernel :244-310).  H_new takes dtype_h (the dtype of H_residual). */
int mhc_add_residual_forward(const void* H_residual, int dtype_h,
                             const void* branch_output, int dtype_bo,
                             const float* H_post, void* H_new,
                             int64_t B, int64_t S, int64_t D, mhc_stream_t stream);

size_t mhc_add_residual_backward_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype_h);

/* Replaces add_residual_backward (reference src/mhc/_backward.py:533-575,
 * kernel :269-351, plus the .sum at :573).  The identity gradient
 * dH_residual = dH_new is not copied: callers alias it.
 *   d_bo[b,s,:]  = sum_n H_post[b,n] dH_new[b,s,n,:]     (dtype_bo)
 *   dH_post[b,n] = sum_{s,d} dH_new[b,s,n,:] * bo[b,s,:]  (f32) */
int mhc_add_residual_backward(const void* dH_new, int dtype_h,
                              const void* branch_output, int dtype_bo,
                              const float* H_post, void* d_branch_output, float* dH_post,
                              int64_t B, int64_t S, int64_t D,
                              void* workspace, size_t workspace_bytes,
                              mhc_stream_t stream);

/* ------------------------------------------------------------------------
 * Dynamic weights (Eq. 14-19) over R rows of x [R,K]:
 *   raw = x @ phi, inv_rms = 1/sqrt(sum(x^2)/K + eps),
 *   s = inv_rms * alpha_g * raw + bias,
 *   H_pre = sigmoid(s[0:4]) / (sum + eps), H_post = 2 sigmoid(s[4:8]),
 *   H_res = Sinkhorn(|s[8:24]| + eps, iters, eps).
 * phi is the API layout [K,24] (no transposed copy); alpha_* point to one
 * f32 each on the device (no host synchronisation).
 * ------------------------------------------------------------------------ */

size_t mhc_dynamic_weights_workspace_bytes(int64_t R, int64_t K);

/* Replaces fused_dynamic_weights_forward (reference src/mhc/_kernels.py:690-752,
 * kernel :318-590) and the alpha .item() syncs of ops.py:96-100.
 * aux [R,25] f32 (optional, may be NULL) receives raw[0:24] and inv_rms for
 * the backward. */
int mhc_dynamic_weights_forward(const void* x, int dtype_x, const float* phi, const float* bias,
                                const float* alpha_pre, const float* alpha_post,
                                const float* alpha_res,
                                float* H_pre, float* H_post, float* H_res, float* aux,
                                int64_t R, int64_t K, int iters, float eps,
                                void* workspace, size_t workspace_bytes,
                                mhc_stream_t stream);

size_t mhc_dynamic_weights_backward_workspace_bytes(int64_t R, int64_t K);

/* Replaces the torch backward of _FusedDynamicWeights (reference
 * src/mhc/ops.py:110-228, Sinkhorn part via _backward.py:503).
 * aux is the forward's aux output.  grad_x [R,K] is written in dtype_x (the
 * dtype the reference's backward casts it back to, ops.py:218-228); the
 * parameter gradients are f32: grad_phi [K,24], grad_bias [24],
 * grad_alpha [3] (pre, post, res). */
int mhc_dynamic_weights_backward(const void* x, int dtype_x, const float* phi, const float* bias,
                                 const float* alpha_pre, const float* alpha_post,
                                 const float* alpha_res, const float* aux, const float* H_pre,
                                 const float* grad_H_pre, const float* grad_H_post,
                                 const float* grad_H_res,
                                 void* grad_x, float* grad_phi, float* grad_bias,
                                 float* grad_alpha,
                                 int64_t R, int64_t K, int iters, float eps,
                                 void* workspace, size_t workspace_bytes,
                                 mhc_stream_t stream);

/* ------------------------------------------------------------------------
 * HyperConnection layer path (reference src/mhc/module.py:103-182).
 *
 * The module's forward H.mean(1) -> fused_dynamic_weights -> fused_stream_mix
 * and its closure fused_add_residual are regrouped so that H_residual is never
 * materialised: pass A reads H for the mean, pass B for branch_input, and the
 * closure recomputes H_res @ H while adding H_post * branch_output.  The packed
 * per-batch weights w [B,24] f32 hold H_pre (0:4), H_post (4:8), H_res (8:24).
 * ------------------------------------------------------------------------ */

size_t mhc_layer_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype);

size_t mhc_mean_pool_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype);

/* Mean over the sequence, module.py:123 (H.mean(dim=1).reshape(B, 4D)),
 * accumulated and returned in f32: x [B, 4D].  Two launches: split-S column
 * sums into the workspace, then a fixed-order reduce over the S chunks. */
int mhc_mean_pool(const void* H, int dtype, float* x, int64_t B, int64_t S, int64_t D,
                  void* workspace, size_t workspace_bytes, mhc_stream_t stream);

/* Dynamic layer forward (module.py:119-139 + 177): mean-pool, Eq. 14-19
 * with bias = [H_pre_base, H_post_base, H_res_base], then branch_input.
 * Outputs: branch_input [B,S,D] (dtype), x [B,4D] f32, w [B,24] f32,
 * aux [B,25] f32.  x (the pooled rows, an input of the backward) may be NULL
 * when no backward follows, and at S = 1 whatever follows (the backward then
 * reads H's rows): the pooled rows are then not kept (and at S = 1 with many
 * batches not formed at all). */
int mhc_layer_dynamic_forward(const void* H, int dtype, const float* phi,
                              const float* H_pre_base, const float* H_post_base,
                              const float* H_res_base, const float* alpha_pre,
                              const float* alpha_post, const float* alpha_res,
                              void* branch_input, float* x, float* w, float* aux,
                              int64_t B, int64_t S, int64_t D, int iters, float eps,
                              void* workspace, size_t workspace_bytes, mhc_stream_t stream);

/* Size of the static device scratch of mhc_layer_dynamic_forward_noalloc
 * (16 MiB, held by every GPU the library runs on until the process ends). */
#define MHC_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): mhc_layer_dynamic_forward with the same arguments, outputs
 * and bits, but no workspace argument.  Its scratch (the mean-pool column
 * partials and the projection partials) is a static device array of
 * MHC_NOALLOC_SCRATCH_BYTES; the call allocates nothing.  It returns
 * MHC_ERR_WORKSPACE, before any device work, when the shape needs more:
 * about 17.6 * B * D bytes once that exceeds 3 MiB (6 MiB for fp32 H), so
 * B * D up to about 950k fits (B = 232 at D = 4096, any S).  The scratch
 * starts from nothing it has to find zeroed: each call overwrites every entry
 * it reads.  All calls on one GPU share that GPU's array, so calls that overlap
 * on one GPU (on different streams) race; serialise them.  The array's address
 * is looked up on the first call on each GPU and kept for the process: once
 * this entry point has run on a GPU, do not call it there again after
 * hipDeviceReset (which unloads the code object the address points into).
 * With x NULL, S > 1 and B * D of 2^19 or more (B >= 64) its weights can
 * differ in their last bits from the workspace entry's: it has no room to keep
 * the pooled rows for their projection, and folds the projection into the
 * mean-pool instead. */
int mhc_layer_dynamic_forward_noalloc(const void* H, int dtype, const float* phi,
                                      const float* H_pre_base, const float* H_post_base,
                                      const float* H_res_base, const float* alpha_pre,
                                      const float* alpha_post, const float* alpha_res,
                                      void* branch_input, float* x, float* w, float* aux,
                                      int64_t B, int64_t S, int64_t D, int iters, float eps,
                                      mhc_stream_t stream);

/* Static layer forward (module.py:108-117 + 177): w from the base
 * parameters (H_post = sigmoid, H_pre = sigmoid/(sum+1e-8), H_res = Sinkhorn
 * with eps 1e-8), then branch_input. */
int mhc_layer_static_forward(const void* H, int dtype, const float* H_pre_base,
                             const float* H_post_base, const float* H_res_base,
                             void* branch_input, float* w,
                             int64_t B, int64_t S, int64_t D, int iters,
                             mhc_stream_t stream);

/* branch_input[b,s,:] = sum_n w[b,n] H[b,s,n,:] from packed weights w [B,24]
 * (module.py:177 for weights computed outside the library, the unfused
 * dynamic path module.py:141-163). */
int mhc_layer_branch_input(const void* H, int dtype, const float* w, void* branch_input,
                           int64_t B, int64_t S, int64_t D, mhc_stream_t stream);

/* Backward of branch_input and of the closure's H_res @ H for packed weights w:
 *   dH = H_pre d_bi + H_res^T dH_new (dH may be NULL, dH_new may be NULL),
 *   dH_pre [B,4] = sum d_bi * H[n], dH_res [B,16] = sum dH_new[n] * H[m]  (f32). */
int mhc_layer_mix_backward(const void* H, int dtype, const void* d_branch_input, const void* dH_new,
                           const float* w, void* dH, float* dH_pre, float* dH_res,
                           int64_t B, int64_t S, int64_t D,
                           void* workspace, size_t workspace_bytes, mhc_stream_t stream);

/* dH of a layer whose weights w [B,24] come from the caller's own ops (the
 * unfused dynamic path, module.py:141-163), with the sequence mean's share
 * folded in:  dH[b,s,m,:] = H_pre[m] d_bi + sum_n H_res[n,m] dH_new[n]
 *                          + grad_x[b, m*D:(m+1)*D] / S,
 * where grad_x [B,4D] f32 is the gradient of x = H.mean(1).reshape(B, 4D)
 * (module.py:123).  One pass, rounded once to dtype; replaces the mix
 * backward's dH plus autograd's broadcast add of the mean's gradient.
 * dH_new may be NULL (H_new received no gradient). */
int mhc_layer_mix_dh(const void* d_branch_input, const void* dH_new, int dtype, const float* w,
                     const float* grad_x, void* dH, int64_t B, int64_t S, int64_t D,
                     mhc_stream_t stream);

/* Layer closure forward (module.py:179-180 with H_residual recomputed):
 * H_new[n] = sum_m H_res[n,m] H[m] + H_post[n] bo, H_new in dtype_h. */
int mhc_layer_add_forward(const void* H, int dtype_h, const void* branch_output, int dtype_bo,
                          const float* w, void* H_new, int64_t B, int64_t S, int64_t D,
                          mhc_stream_t stream);

/* Layer closure backward: d_bo = sum_n H_post[n] dH_new[n] (dtype_bo) and
 * dH_post [B,4] f32. */
int mhc_layer_add_backward(const void* dH_new, int dtype_h, const void* branch_output,
                           int dtype_bo, const float* w, void* d_branch_output, float* dH_post,
                           int64_t B, int64_t S, int64_t D,
                           void* workspace, size_t workspace_bytes, mhc_stream_t stream);

/* Dynamic layer backward: given d_bi [B,S,D], dH_new [B,S,4,D] (NULL when
 * H_new received no gradient) and dH_post [B,4] f32 from the closure backward,
 * writes dH [B,S,4,D] (NULL to skip) and the f32 parameter gradients
 * grad_phi [4D,24], grad_bias [24] (pre, post, res), grad_alpha [3].  x is the
 * forward's pooled rows; at S = 1 it may be NULL (the forward then need not
 * write it): the pooled rows are H's own rows, read from H.  With B = 0 the
 * parameter gradients are zero (empty sums). */
int mhc_layer_dynamic_backward(const void* H, int dtype, const void* d_branch_input,
                               const void* dH_new, const float* dH_post,
                               const float* phi, const float* H_pre_base,
                               const float* H_post_base, const float* H_res_base,
                               const float* alpha_pre, const float* alpha_post,
                               const float* alpha_res, const float* x, const float* w,
                               const float* aux, void* dH, float* grad_phi, float* grad_bias,
                               float* grad_alpha, int64_t B, int64_t S, int64_t D, int iters,
                               float eps, void* workspace, size_t workspace_bytes,
                               mhc_stream_t stream);

/* Static layer backward: dH (NULL to skip) and grad_bias [24] f32 for
 * (H_pre_base, H_post_base, H_res_base); zero with B = 0. */
int mhc_layer_static_backward(const void* H, int dtype, const void* d_branch_input,
                              const void* dH_new, const float* dH_post,
                              const float* H_pre_base, const float* H_post_base,
                              const float* H_res_base, const float* w, void* dH,
                              float* grad_bias, int64_t B, int64_t S, int64_t D, int iters,
                              void* workspace, size_t workspace_bytes, mhc_stream_t stream);

/* ------------------------------------------------------------------------
 * The two ends of a hyper-connection stack.  No counterpart in the
 * reference, which takes the hyper-hidden state (batch, seq, 4, dim) as
 * given (README.md:38-39) and leaves building it from the embeddings, and
 * reducing it at the model output, to the caller.  Each is the other's
 * backward with the same scale (they are adjoint), so two entry points
 * cover both passes.
 * Accumulation is f32; x, y and H may have different dtypes.
 * ------------------------------------------------------------------------ */

/* H[b,s,n,:] = scale * x[b,s,:] for n = 0..3.  x [B,S,D] (dtype_x),
 * H [B,S,4,D] (dtype_h).  Backward of stream_collapse. */
int mhc_stream_expand(const void* x, int dtype_x, void* H, int dtype_h, int64_t B, int64_t S,
                      int64_t D, float scale, mhc_stream_t stream);

/* y[b,s,:] = scale * sum_n H[b,s,n,:] (scale 1 = sum, 1/4 = mean).  H [B,S,4,D]
 * (dtype_h), y [B,S,D] (dtype_y).  Backward of stream_expand. */
int mhc_stream_collapse(const void* H, int dtype_h, void* y, int dtype_y, int64_t B, int64_t S,
                        int64_t D, float scale, mhc_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_ABI_H */
