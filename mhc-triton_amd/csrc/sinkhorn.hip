// Standalone Sinkhorn-Knopp forward / backward over N independent 4x4
// matrices (reference src/mhc/_kernels.py:30-130,597-614 and
// src/mhc/_backward.py:29-262,503-530).
//
// One matrix per lane: a wave handles 64 matrices, a 256-thread workgroup
// 256.  Each lane reads its 16 entries with 16-byte loads (4 for fp32, 2 for
// bf16/fp16); across the wave the accesses cover one contiguous span.  The
// forward is VALU-bound at 20 rounds (40 VALU ops and 8 v_rcp per round in
// the scaling-vector form of sk_forward); the backward keeps every round's
// scaling vectors in registers for up to 20 rounds and carries the adjoint in
// scaled coordinates (sk_backward_scaled: 95-100 us at 2^20 matrices, 20
// rounds, against 131 us for the explicit normalisation backward on the same
// states and 175 us for the checkpointed reverse sweep).  From 21 to 64
// rounds it recomputes the vectors in 16-round segments from checkpoints
// (sk_backward_segmented; fwd + bwd at 2^20 matrices: 190 against 255 us at
// 21 rounds, 436 against 818 us at 64); past 64 rounds it keeps the
// checkpointed sweep.  The unaligned (element-wise load) path runs the same
// forms (fwd + bwd at 20 rounds: 130-134 against 241-245 us with the
// checkpointed sweep it used before).
#include "sinkhorn.hpp"

namespace mhc {

template <typename T, bool VEC>
__device__ __forceinline__ void load_mat(const T* p, float (&m)[16]) {
  if constexpr (VEC) {
    constexpr int N = Vec<T>::N;
#pragma unroll
    for (int q = 0; q < 16 / N; ++q) Io<T>::load(p + q * N, m + q * N);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) m[k] = to_f32(p[k]);
  }
}

template <typename T, bool VEC>
__device__ __forceinline__ void store_mat(T* p, const float (&m)[16]) {
  if constexpr (VEC) {
    constexpr int N = Vec<T>::N;
#pragma unroll
    for (int q = 0; q < 16 / N; ++q) Io<T>::template store<false>(p + q * N, m + q * N);
  } else {
#pragma unroll
    for (int k = 0; k < 16; ++k) p[k] = from_f32<T>(m[k]);
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kThreads) void sinkhorn_fwd_kernel(const T* __restrict__ M, T* __restrict__ out,
                                                                int64_t n, int iters, float eps) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  float m[16];
  load_mat<T, VEC>(M + i * 16, m);
  sk_forward(m, iters, eps);
  store_mat<T, VEC>(out + i * 16, m);
}

constexpr int kSkScaledMax = 20;  // rounds the scaling-vector backward keeps in registers
constexpr int kSkSegRounds = 16;  // rounds per segment of the segmented backward
constexpr int kSkSegs = 4;        // its segments: up to 64 rounds

template <typename T, typename TD, bool VEC>
__global__ __launch_bounds__(kThreads) void sinkhorn_bwd_kernel(const T* __restrict__ M, const TD* __restrict__ dP,
                                                                T* __restrict__ dM, int64_t n, int iters, float eps) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  float m[16], d[16];
  load_mat<T, VEC>(M + i * 16, m);
  load_mat<TD, VEC>(dP + i * 16, d);
  // Past 64 rounds the explicit-state checkpoints: on the unaligned path five
  // keep 3 waves per SIMD (its element-wise loads need more registers; ten
  // would leave one).  The result does not depend on the checkpoint count.
  if (iters <= kSkScaledMax)
    sk_backward_scaled<kSkScaledMax>(m, d, iters, eps);
  else if (iters <= kSkSegRounds * kSkSegs)
    sk_backward_segmented<kSkSegRounds, kSkSegs>(m, d, iters, eps);
  else
    sk_backward<VEC ? 10 : 5>(m, d, iters, eps);
  store_mat<T, VEC>(dM + i * 16, d);
}

static int check_common(int64_t n_mat, int iters) {
  if (n_mat < 0) { set_error("sinkhorn: negative matrix count %lld", (long long)n_mat); return MHC_ERR_ARG; }
  if (iters < 0) { set_error("sinkhorn: negative iteration count %d", iters); return MHC_ERR_ARG; }
  return MHC_OK;
}

}  // namespace mhc

using namespace mhc;

extern "C" int mhc_sinkhorn_forward(const void* M, void* out, int64_t n_mat, int dtype, int iters, float eps,
                                    mhc_stream_t stream) {
  if (int rc = check_common(n_mat, iters)) return rc;
  if (n_mat == 0) return MHC_OK;
  if (!M || !out) { set_error("sinkhorn_forward: null pointer"); return MHC_ERR_ARG; }
  const bool vec = aligned16(M) && aligned16(out);
  const dim3 grid((unsigned)((n_mat + kThreads - 1) / kThreads));
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    if (vec)
      sinkhorn_fwd_kernel<T, true><<<grid, kThreads, 0, (hipStream_t)stream>>>(
          (const T*)M, (T*)out, n_mat, iters, eps);
    else
      sinkhorn_fwd_kernel<T, false><<<grid, kThreads, 0, (hipStream_t)stream>>>(
          (const T*)M, (T*)out, n_mat, iters, eps);
    return hip_status(hipGetLastError(), "sinkhorn_forward launch");
  });
}

extern "C" int mhc_sinkhorn_backward(const void* M, int dtype_M, const void* dP, int dtype_dP, void* dM,
                                     int64_t n_mat, int iters, float eps, mhc_stream_t stream) {
  if (int rc = check_common(n_mat, iters)) return rc;
  if (n_mat == 0) return MHC_OK;
  if (!M || !dP || !dM) { set_error("sinkhorn_backward: null pointer"); return MHC_ERR_ARG; }
  const bool vec = aligned16(M) && aligned16(dP) && aligned16(dM);
  const dim3 grid((unsigned)((n_mat + kThreads - 1) / kThreads));
  return MHC_DISPATCH_DTYPE(dtype_M, [&] {
    using TM = T;
    return MHC_DISPATCH_DTYPE(dtype_dP, [&] {
      if (vec)
        sinkhorn_bwd_kernel<TM, T, true><<<grid, kThreads, 0, (hipStream_t)stream>>>(
            (const TM*)M, (const T*)dP, (TM*)dM, n_mat, iters, eps);
      else
        sinkhorn_bwd_kernel<TM, T, false><<<grid, kThreads, 0, (hipStream_t)stream>>>(
            (const TM*)M, (const T*)dP, (TM*)dM, n_mat, iters, eps);
      return hip_status(hipGetLastError(), "sinkhorn_backward launch");
    });
  });
}
