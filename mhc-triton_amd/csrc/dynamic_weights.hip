// Entry points: fused_dynamic_weights forward / backward and the sequence
// mean-pool (reference src/mhc/_kernels.py:690-752, src/mhc/ops.py:72-228,
// src/mhc/module.py:123).
#include "dynw_kernels.hpp"
#include "stream_kernels.hpp"

namespace mhc {

int check_workspace(const char* who, const void* ws, size_t have, size_t need);

constexpr int kRT = 4;  // rows per workgroup in dynw_partial_kernel

struct DynPlan {
  int64_t KC;  // K chunk per workgroup (multiple of 256)
  int nK;      // number of chunks
};

// Aim for at most ~4096 workgroups: small R splits K finely (R = 4, K = 16384
// -> 64 chunks of 256), large R gives each workgroup a longer K run.
static DynPlan dyn_plan(int64_t R, int64_t K) {
  const int64_t rtiles = (R + kRT - 1) / kRT;
  const int64_t k256 = (K + kThreads - 1) / kThreads;
  int64_t kpt = (rtiles * k256 + 4095) / 4096;
  if (kpt < 1) kpt = 1;
  if (kpt > 64) kpt = 64;
  DynPlan p;
  p.KC = kThreads * kpt;
  p.nK = (int)((K + p.KC - 1) / p.KC);
  if (p.nK < 1) p.nK = 1;
  return p;
}

static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// MFMA plan for x with many rows (dynw_mfma_kernel): K chunks of
// mfma_steps(esize) * kMfmaWaves steps (1024 k for 16-bit x, 512 k for fp32),
// and row ranges of whole 32-row tiles so that about kMfmaTargetWg workgroups
// run, one per CU (the kernel's LDS allows one).
// At R = K = 16384, 16-bit x: 16 chunks x 16 ranges of 1024 rows.
constexpr int64_t kMfmaMinRows = 64;
constexpr int64_t kMfmaTargetWg = 256;

struct MfmaPlan {
  int64_t nsteps;       // K / 16
  int nK;               // chunks
  int64_t rows_per_wg;  // multiple of 32
  int ngr;              // row ranges
  size_t part_bytes;
};

static bool mfma_shape_ok(int64_t R, int64_t K, int esize) {
  return R >= kMfmaMinRows && K > 0 && K % 16 == 0 && span_ok(32 * K, esize) && span_ok(K * kOut, 4);
}

static MfmaPlan mfma_plan(int64_t R, int64_t K, int esize) {
  MfmaPlan p;
  const int64_t chunk_steps = (int64_t)kMfmaWaves * mfma_steps(esize);
  p.nsteps = K / 16;
  p.nK = (int)((p.nsteps + chunk_steps - 1) / chunk_steps);
  if (p.nK < 1) p.nK = 1;
  const int64_t tiles = (R + 31) / 32;
  int64_t ngr = (kMfmaTargetWg + p.nK - 1) / p.nK;
  if (ngr > tiles) ngr = tiles;
  if (ngr < 1) ngr = 1;
  int64_t tpw = (tiles + ngr - 1) / ngr;
  while (tpw > 1 && !span_ok(32 * tpw * K, esize)) tpw = (tpw + 1) / 2;
  p.rows_per_wg = 32 * tpw;
  p.ngr = (int)((R + p.rows_per_wg - 1) / p.rows_per_wg);
  p.part_bytes = align256((size_t)R * p.nK * kPart * sizeof(float));
  return p;
}

}  // namespace mhc

using namespace mhc;

// The largest of the two plans (the dtype and alignment that pick the plan are
// not arguments of the query).
extern "C" size_t mhc_dynamic_weights_workspace_bytes(int64_t R, int64_t K) {
  if (R <= 0) return 0;
  const DynPlan p = dyn_plan(R, K);
  size_t need = align256((size_t)R * p.nK * kPart * sizeof(float));
  for (int esize : {2, 4})
    if (mfma_shape_ok(R, K, esize)) {
      const MfmaPlan m = mfma_plan(R, K, esize);
      if (m.part_bytes > need) need = m.part_bytes;
    }
  return need;
}

extern "C" int mhc_dynamic_weights_forward(const void* x, int dtype_x, const float* phi, const float* bias,
                                           const float* alpha_pre, const float* alpha_post,
                                           const float* alpha_res, float* H_pre, float* H_post, float* H_res,
                                           float* aux, int64_t R, int64_t K, int iters, float eps,
                                           void* workspace, size_t workspace_bytes, mhc_stream_t stream) {
  if (R < 0 || K < 0 || iters < 0) {
    set_error("dynamic_weights_forward: bad size (R=%lld K=%lld iters=%d)", (long long)R, (long long)K, iters);
    return MHC_ERR_ARG;
  }
  if (R == 0) return MHC_OK;
  if (!x || !phi || !bias || !alpha_pre || !alpha_post || !alpha_res || !H_pre || !H_post || !H_res) {
    set_error("dynamic_weights_forward: null pointer");
    return MHC_ERR_ARG;
  }
  if (int rc = check_workspace("dynamic_weights_forward", workspace, workspace_bytes,
                               mhc_dynamic_weights_workspace_bytes(R, K)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  int nK = 0;
  const int esize = dtype_x == MHC_DTYPE_F32 ? 4 : 2;
  if (mfma_shape_ok(R, K, esize) && aligned16(x)) {
    // rows in bulk: the projection on MFMA (HBM-bound instead of VALU-bound).
    const MfmaPlan m = mfma_plan(R, K, esize);
    const dim3 grid((unsigned)m.ngr, (unsigned)m.nK);
    int rc = MHC_DISPATCH_DTYPE(dtype_x, [&] {
      dynw_mfma_kernel<T><<<grid, 64 * kMfmaWaves, 0, st>>>((const T*)x, phi, part, R, K, m.nK, m.rows_per_wg);
      return hip_status(hipGetLastError(), "dynamic_weights_forward mfma launch");
    });
    if (rc) return rc;
    nK = m.nK;
  } else {
    const DynPlan p = dyn_plan(R, K);
    const bool phi_vec = aligned16(phi);
    int rc = MHC_DISPATCH_DTYPE(dtype_x, [&] {
      dynw_partial_kernel<T, kRT><<<dim3((unsigned)((R + kRT - 1) / kRT), p.nK), kThreads, 0, st>>>(
          (const T*)x, phi, part, R, K, p.nK, p.KC, phi_vec);
      return hip_status(hipGetLastError(), "dynamic_weights_forward partial launch");
    });
    if (rc) return rc;
    nK = p.nK;
  }
  DynParams P{bias, bias + 4, bias + 8, alpha_pre, alpha_post, alpha_res};
  if (R >= kMfmaMinRows && nK <= 64)
    dynw_finalize_rows_kernel<><<<dim3((unsigned)((R + kFinRowsWg - 1) / kFinRowsWg)), kThreads, 0, st>>>(
        part, nK, R, K, P, OutRow{H_pre, 4}, OutRow{H_post, 4}, OutRow{H_res, 16}, aux, iters, eps);
  else
    dynw_finalize_kernel<><<<dim3((unsigned)((R + 3) / 4)), kThreads, 0, st>>>(
        part, nK, R, K, P, OutRow{H_pre, 4}, OutRow{H_post, 4}, OutRow{H_res, 16}, aux, iters, eps);
  return hip_status(hipGetLastError(), "dynamic_weights_forward finalize launch");
}

namespace mhc {

// The layer path at many batches: rows x [R, K] (the pooled rows in fp32, or at S = 1 H's own
// rows) projected on the MFMA kernel into the partial records part[R][nK][25], as the op does
// for rows in bulk.
bool dynw_project_rows_ok(int64_t R, int64_t K, const void* x, int dtype) {
  return mfma_shape_ok(R, K, dtype == MHC_DTYPE_F32 ? 4 : 2) && aligned16(x);
}

int dynw_project_rows(const void* x, int dtype, const float* phi, float* part, int64_t R, int64_t K, int* nK,
                      hipStream_t st) {
  const MfmaPlan m = mfma_plan(R, K, dtype == MHC_DTYPE_F32 ? 4 : 2);
  *nK = m.nK;
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    dynw_mfma_kernel<T><<<dim3((unsigned)m.ngr, (unsigned)m.nK), 64 * kMfmaWaves, 0, st>>>(
        (const T*)x, phi, part, R, K, m.nK, m.rows_per_wg);
    return hip_status(hipGetLastError(), "layer projection mfma launch");
  });
}

}  // namespace mhc

// Row chunks of the backward's wide pass: one chunk for a batch's worth of
// rows; for many rows about 1024 workgroups, at least 64 rows each.
struct WidePlan {
  int64_t RC;  // rows per chunk
  int nR;      // chunks
};

static WidePlan wide_plan(int64_t R, int64_t K) {
  WidePlan p;
  const int64_t ncol = K > 0 ? (K + kThreads - 1) / kThreads : 1;
  int64_t nr = (1024 + ncol - 1) / ncol;
  const int64_t max_nr = (R + 63) / 64;
  if (nr > max_nr) nr = max_nr;
  if (nr < 1) nr = 1;
  p.RC = (R + nr - 1) / nr;
  if (p.RC < 1) p.RC = 1;
  p.nR = (int)((R + p.RC - 1) / p.RC);
  if (p.nR < 1) p.nR = 1;
  return p;
}

// Row chunks of the MFMA backward (dynw_bwd_mfma_kernel, any x dtype): one 8-wave workgroup
// fits a CU, so about kMfmaTargetWg workgroups, each walking a long chunk: its
// pipeline fills and drains once per chunk, and fewer chunks leave fewer grad_phi
// partials.  At R = K = 16384, 4 chunks of 4096 rows (256 workgroups) took
// 179-181 us against 199-203 us for 16 (1024 workgroups) and 223-224 us for 32.
// Never more chunks than the wide plan w (whose workspace holds the partials);
// chunks are split further while a chunk's buffer spans (esize-byte x or grad_x
// elements) would pass 2^31 bytes.
static WidePlan mfma_bwd_plan(int64_t R, int64_t K, const WidePlan& w, int esize) {
  const int64_t ncb = (K + 32 * kBwdWaves - 1) / (32 * kBwdWaves);
  int64_t nr = (kMfmaTargetWg + ncb - 1) / ncb;
  if (nr > w.nR) nr = w.nR;
  for (;;) {
    WidePlan p;
    p.RC = (R + nr - 1) / nr;
    p.nR = (int)((R + p.RC - 1) / p.RC);
    const int64_t span_rows = p.RC + 4 * kBwdRows;
    if (nr >= w.nR || (span_ok(span_rows * K, esize) && span_ok(span_rows * kRow, 4))) return nr >= w.nR ? w : p;
    nr = 2 * nr < w.nR ? 2 * nr : w.nR;
  }
}

namespace mhc {

// Workspace of dynw_grad_pass with split rows: the grad_phi chunk partials, and the grad_bias /
// grad_alpha chunk records (none with one chunk).
size_t dynw_grad_split_bytes(int64_t R, int64_t K) {
  const WidePlan w = wide_plan(R, K);
  if (w.nR <= 1) return 0;
  return align256((size_t)w.nR * K * kOut * sizeof(float)) + align256((size_t)w.nR * 27 * sizeof(float));
}

// grad_x, grad_phi, grad_bias and grad_alpha from the per-row records rowbuf [R][kRow] that
// dynw_bwd_rows_kernel wrote: rows in bulk on the MFMA kernel, else the VALU wide pass, in row
// chunks whose grad_phi / bias partials dynw_gphi_reduce_kernel then adds in chunk order.
// grad_x is in x's dtype, or f32 with gx_f32 (the layer at S = 1 passes H's rows as x).
// split_ws holds dynw_grad_split_bytes(R, K) bytes.
int dynw_grad_pass(const void* x, int dtype_x, const float* phi, const float* rowbuf, void* grad_x, bool gx_f32,
                   float* grad_phi, float* grad_bias, float* grad_alpha, int64_t R, int64_t K, char* split_ws,
                   hipStream_t st) {
  const bool phi_vec = aligned16(phi);
  const WidePlan w = wide_plan(R, K);
  const int esize = dtype_x == MHC_DTYPE_F32 ? 4 : 2;
  const int span_esize = gx_f32 && grad_x ? 4 : esize;  // the wider of x and grad_x
  const bool mfma_ok = R >= kMfmaMinRows && K > 0 && K % (16 / esize) == 0 && aligned16(x) &&
                       (!grad_x || aligned16(grad_x));
  // the row chunks of the pass that runs (the MFMA plan has at most w.nR)
  const WidePlan pl = mfma_ok ? mfma_bwd_plan(R, K, w, span_esize) : w;
  float* gphi_part = (pl.nR > 1 && grad_phi) ? (float*)split_ws : nullptr;
  float* bias_part = nullptr;  // MFMA path, split rows: per-chunk grad_bias / grad_alpha records
  int rc;
  // (the kernel's buffer spans reach up to four blocks past a chunk's rows)
  if (mfma_ok && span_ok((pl.RC + 4 * kBwdRows) * K, span_esize) && span_ok((pl.RC + 4 * kBwdRows) * kRow, 4)) {
    // rows in bulk: grad_x and grad_phi on MFMA.
    if (pl.nR > 1 && (grad_bias || grad_alpha))
      bias_part = (float*)(split_ws + align256((size_t)w.nR * K * kOut * sizeof(float)));
    const dim3 grid((unsigned)((K + 32 * kBwdWaves - 1) / (32 * kBwdWaves)), (unsigned)pl.nR);
    // Chunks of one 64-row block load it alone: with 16-bit x and grad_x, loads of the next
    // block (out of range) in flight as well cost 1.3-2.2 us at R = 64-256, K = 16384; from two
    // blocks on the two ahead time alike, from six (R = 1536) they win by 1.6-2.6 us.
    rc = MHC_DISPATCH_DTYPE(dtype_x, [&] {
      if (gx_f32)
        dynw_bwd_mfma_kernel<T, float><<<grid, 64 * kBwdWaves, 0, st>>>(
            (const T*)x, phi, rowbuf, (float*)grad_x, grad_phi, gphi_part, bias_part, grad_bias, grad_alpha, R, K,
            pl.RC);
      else if (pl.RC <= kBwdRows)
        dynw_bwd_mfma_kernel<T, T, 1><<<grid, 64 * kBwdWaves, 0, st>>>(
            (const T*)x, phi, rowbuf, (T*)grad_x, grad_phi, gphi_part, bias_part, grad_bias, grad_alpha, R, K,
            pl.RC);
      else
        dynw_bwd_mfma_kernel<T><<<grid, 64 * kBwdWaves, 0, st>>>((const T*)x, phi, rowbuf, (T*)grad_x, grad_phi,
                                                                 gphi_part, bias_part, grad_bias, grad_alpha, R,
                                                                 K, pl.RC);
      return hip_status(hipGetLastError(), "dynamic_weights_backward mfma launch");
    });
  } else {
    rc = MHC_DISPATCH_DTYPE(dtype_x, [&] {
      const hipError_t e =
          gx_f32 ? launch_dynw_bwd_wide<T, float>((const T*)x, phi, rowbuf, (float*)grad_x, grad_phi, gphi_part,
                                                  grad_bias, grad_alpha, R, K, pl.RC, (unsigned)pl.nR, phi_vec, st)
                 : launch_dynw_bwd_wide<T, T>((const T*)x, phi, rowbuf, (T*)grad_x, grad_phi, gphi_part, grad_bias,
                                              grad_alpha, R, K, pl.RC, (unsigned)pl.nR, phi_vec, st);
      return hip_status(e, "dynamic_weights_backward wide launch");
    });
  }
  if (rc || (!gphi_part && !bias_part)) return rc;
  const int64_t n = gphi_part ? K * kOut : 0;
  const int64_t nt = n + (bias_part ? 27 : 0);
  dynw_gphi_reduce_kernel<><<<dim3((unsigned)((nt + kThreads - 1) / kThreads)), kThreads, 0, st>>>(
      gphi_part, grad_phi, n, pl.nR, bias_part, grad_bias, grad_alpha);
  return hip_status(hipGetLastError(), "dynamic_weights_backward grad_phi reduce launch");
}

}  // namespace mhc

extern "C" size_t mhc_dynamic_weights_backward_workspace_bytes(int64_t R, int64_t K) {
  if (R <= 0) return 0;
  return align256((size_t)R * kRow * sizeof(float)) + dynw_grad_split_bytes(R, K);
}

extern "C" int mhc_dynamic_weights_backward(const void* x, int dtype_x, const float* phi, const float* bias,
                                            const float* alpha_pre, const float* alpha_post,
                                            const float* alpha_res, const float* aux, const float* H_pre,
                                            const float* grad_H_pre, const float* grad_H_post,
                                            const float* grad_H_res, void* grad_x, float* grad_phi,
                                            float* grad_bias, float* grad_alpha, int64_t R, int64_t K, int iters,
                                            float eps, void* workspace, size_t workspace_bytes,
                                            mhc_stream_t stream) {
  if (R < 0 || K < 0 || iters < 0) {
    set_error("dynamic_weights_backward: bad size (R=%lld K=%lld iters=%d)", (long long)R, (long long)K, iters);
    return MHC_ERR_ARG;
  }
  if (!phi || !bias || !alpha_pre || !alpha_post || !alpha_res) {
    set_error("dynamic_weights_backward: null parameter pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  if (R == 0) {
    // No rows: every gradient is an empty sum.
    if (grad_phi && K > 0)
      if (int rc = fill_zero(grad_phi, K * kOut, st)) return rc;
    if (grad_bias)
      if (int rc = fill_zero(grad_bias, kOut, st)) return rc;
    if (grad_alpha)
      if (int rc = fill_zero(grad_alpha, 3, st)) return rc;
    return MHC_OK;
  }
  if (!x || !aux || !H_pre) {
    set_error("dynamic_weights_backward: null pointer");
    return MHC_ERR_ARG;
  }
  if (int rc = check_workspace("dynamic_weights_backward", workspace, workspace_bytes,
                               mhc_dynamic_weights_backward_workspace_bytes(R, K)))
    return rc;
  float* rowbuf = (float*)workspace;
  DynParams P{bias, bias + 4, bias + 8, alpha_pre, alpha_post, alpha_res};
  // 16 rows per workgroup, four per wave (four rows on wave 0 alone took 11.7 us at R = 16384)
  dynw_bwd_rows_kernel<16><<<dim3((unsigned)((R + 15) / 16)), kThreads, 0, st>>>(
      aux, P, InRow{H_pre, 4}, InRow{grad_H_pre, 4}, InRow{grad_H_post, 4}, InRow{grad_H_res, 16}, nullptr, 0,
      rowbuf, R, K, iters, eps);
  if (int rc = hip_status(hipGetLastError(), "dynamic_weights_backward rows launch")) return rc;
  return dynw_grad_pass(x, dtype_x, phi, rowbuf, grad_x, false, grad_phi, grad_bias, grad_alpha, R, K,
                        (char*)workspace + align256((size_t)R * kRow * sizeof(float)), st);
}

// ---------------------------------------------------------------------------
// Mean-pool
// ---------------------------------------------------------------------------
namespace mhc {

constexpr int kPoolUN = 4;  // rows in flight per lane in colsum_kernel
// Sequences up to this length take colsum_direct_kernel (one launch, the same
// bits): at such lengths the pass is a few microseconds of latency, and the
// second launch and the column-partial round trip are most of it.
constexpr int64_t kPoolDirectRows = 8;

template <typename T, int W, bool PROJ>
static int launch_meanpool(const T* H, float* x, const float* phi, float* projpart, float* colpart, int64_t B,
                           int64_t S, int64_t K, hipStream_t st) {
  const PoolPlan p = pool_plan(B, S, K, W);
  const float inv_S = S > 0 ? 1.f / (float)S : __builtin_nanf("");
  const bool phi_vec = phi ? aligned16(phi) : false;
  for (int64_t b0 = 0; b0 < B; b0 += kMaxGridY) {
    const int64_t nb = (B - b0) < kMaxGridY ? (B - b0) : kMaxGridY;
    // Without the projection, the single launch also serves lengths up to 64 that the plan does
    // not split (one S chunk: enough batches fill the GPU), where the column partials would be x
    // itself (B = 4096, S = 16: 563 -> 419 us; B = 512, S = 64: 242 -> 232).  Longer ones keep
    // colsum_kernel, whose streaming loads read them faster (B = 48, S = 256: 69 against 71 us).
    const bool direct_vec =
        !PROJ && W > 1 && aligned16(x) && (S <= kPoolDirectRows || (p.nS == 1 && S <= 64));
    if (direct_vec || S <= kPoolDirectRows) {
      if (direct_vec)
        colsum_direct_vec_kernel<T, W><<<dim3((unsigned)p.ncc, (unsigned)nb), kThreads, 0, st>>>(
            H, x, S, K, p.SC, inv_S, b0);
      else
        colsum_direct_kernel<T, PROJ><<<dim3((unsigned)p.nrc, (unsigned)nb), kThreads, 0, st>>>(
            H, x, phi, projpart, S, K, p.SC, inv_S, b0, phi_vec);
      if (int rc = hip_status(hipGetLastError(), "mean_pool direct launch")) return rc;
      continue;
    }
    // The first half of each S chunk with nt loads, the second half plain: in
    // the layer, branch_input reads H next and finds the chunk tails in the
    // memory-side cache (colsum + branch_input: -4 us at config-3 size, -6 us
    // at config 4, against all plain).
    colsum_kernel<T, W, kPoolUN><<<dim3((unsigned)p.ncc, (unsigned)p.nS, (unsigned)nb), kThreads, 0, st>>>(
        H, colpart, S, K, p.SC, p.nS, p.SC / 2, b0);
    if (int rc = hip_status(hipGetLastError(), "mean_pool column-sum launch")) return rc;
    colsum_reduce_kernel<PROJ><<<dim3((unsigned)p.nrc, (unsigned)nb), kThreads, 0, st>>>(
        colpart, x, phi, projpart, K, p.nS, inv_S, b0, phi_vec);
    if (int rc = hip_status(hipGetLastError(), "mean_pool reduce launch")) return rc;
  }
  return MHC_OK;
}

static bool pool_vec(int dtype, int64_t K, const void* H) {
  const int W = dtype == MHC_DTYPE_F32 ? 4 : 8;
  return K % W == 0 && aligned16(H) && span_ok(kPoolUN * K, 4);
}

PoolPlan mean_pool_plan(int dtype, int64_t B, int64_t S, int64_t D, const void* H) {
  const int64_t K = 4 * D;
  const int W = (H == nullptr || pool_vec(dtype, K, H)) ? (dtype == MHC_DTYPE_F32 ? 4 : 8) : 1;
  return pool_plan(B, S, K, W);
}

// Column-partial workspace of the mean-pool: the largest plan over the vector
// and scalar paths (the scalar path has more, narrower column chunks but the
// same S split or a finer one).
size_t mean_pool_colpart_bytes(int dtype, int64_t B, int64_t S, int64_t D) {
  const int64_t K = 4 * D;
  size_t best = 0;
  for (int W : {dtype == MHC_DTYPE_F32 ? 4 : 8, 1}) {
    const PoolPlan p = pool_plan(B, S, K, W);
    const size_t v = (size_t)B * p.nS * K * sizeof(float);
    if (v > best) best = v;
  }
  return best;
}

// x [B, 4D] f32 (and with phi, the projection partials [B][nrc][25]); returns
// the number of projection chunks through *nrc.
int mean_pool_any(const void* H, int dtype, float* x, const float* phi, float* projpart, float* colpart,
                  int64_t B, int64_t S, int64_t D, int* nrc, hipStream_t st) {
  const int64_t K = 4 * D;
  const bool vec = pool_vec(dtype, K, H);
  if (nrc) *nrc = (int)pool_plan(B, S, K, 1).nrc;
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    constexpr int WV = Vec<T>::N;
    if (phi) {
      if (vec) return launch_meanpool<T, WV, true>((const T*)H, x, phi, projpart, colpart, B, S, K, st);
      return launch_meanpool<T, 1, true>((const T*)H, x, phi, projpart, colpart, B, S, K, st);
    }
    if (vec) return launch_meanpool<T, WV, false>((const T*)H, x, nullptr, nullptr, colpart, B, S, K, st);
    return launch_meanpool<T, 1, false>((const T*)H, x, nullptr, nullptr, colpart, B, S, K, st);
  });
}

static size_t al256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace mhc

extern "C" size_t mhc_mean_pool_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype) {
  if (B <= 0 || D <= 0) return 0;
  return al256(mean_pool_colpart_bytes(dtype, B, S, D));
}

extern "C" int mhc_mean_pool(const void* H, int dtype, float* x, int64_t B, int64_t S, int64_t D, void* workspace,
                             size_t workspace_bytes, mhc_stream_t stream) {
  if (int rc = check_bsd("mean_pool", B, S, D)) return rc;
  if (B * D == 0) return MHC_OK;
  if (!H || !x) {
    set_error("mean_pool: null pointer");
    return MHC_ERR_ARG;
  }
  if (dtype != MHC_DTYPE_F32 && dtype != MHC_DTYPE_BF16 && dtype != MHC_DTYPE_F16) {
    set_error("unsupported dtype code %d", dtype);
    return MHC_ERR_DTYPE;
  }
  if (int rc = check_workspace("mean_pool", workspace, workspace_bytes, mhc_mean_pool_workspace_bytes(B, S, D, dtype)))
    return rc;
  return mean_pool_any(H, dtype, x, nullptr, nullptr, (float*)workspace, B, S, D, nullptr, (hipStream_t)stream);
}
