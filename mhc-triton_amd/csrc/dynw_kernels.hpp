// Dynamic-weight kernels (Eq. 14-19) and the sequence mean-pool.
//
// Forward, standalone op (reference src/mhc/_kernels.py:318-590,690-752):
//   dynw_partial_kernel   split-K partial dot products x[r,:] . phi[:,j] (24)
//                         and sum(x^2) for a tile of RT rows and a K chunk,
//                         reading phi in its API layout [K,24]: one 96-byte
//                         row per k, contiguous across lanes (no transpose).
//   dynw_finalize_kernel  per row: fixed-order sum of the K-chunk partials,
//                         inv_rms, scale + bias, sigmoid / normalise, 2*sigmoid
//                         and the register-resident Sinkhorn of H_res.
// Layer path: colsum_reduce_kernel<PROJ=true> produces the same 25 partials
// per column chunk while it finishes the sequence mean, so the projection
// costs no extra pass over HBM.
//
// Backward (reference src/mhc/_kernels.py ops.py:110-228):
//   dynw_bwd_rows_kernel  per row: Sinkhorn backward, sigmoid / normalise
//                         backward, grad_raw, the rms coefficient and the
//                         per-row bias / alpha contributions.
//   dynw_bwd_wide_kernel  per k: grad_x[r,k] = grad_raw[r,:] . phi[k,:] + coef[r] x[r,k]
//                         and grad_phi[k,:] = sum_r x[r,k] grad_raw[r,:].
//   dynw_bwd_sum_kernel   grad_bias and grad_alpha: fixed-order sums over rows.
#pragma once

#include "sinkhorn.hpp"

namespace mhc {

constexpr int kOut = 24;   // n^2 + 2n outputs of the projection
constexpr int kPart = 25;  // 24 dot products + sum of squares
constexpr int kRow = 52;   // per-row backward record (see dynw_bwd_rows_kernel)

struct OutRow {
  float* p;
  int64_t stride;
};

struct InRow {
  const float* p;
  int64_t stride;
};

__device__ __forceinline__ void load_phi_row(const float* __restrict__ phi, int64_t k, bool vec, float (&ph)[kOut]) {
  const float* p = phi + k * kOut;
  if (vec) {
#pragma unroll
    for (int q = 0; q < 6; ++q) {
      f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * q);
      ph[4 * q] = v.x; ph[4 * q + 1] = v.y; ph[4 * q + 2] = v.z; ph[4 * q + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < kOut; ++j) ph[j] = p[j];
  }
}

// part[r][kc][0:24] = sum_{k in chunk kc} x[r,k] phi[k,:],  part[r][kc][24] = sum x[r,k]^2
template <typename TX, int RT>
__global__ __launch_bounds__(kThreads) void dynw_partial_kernel(const TX* __restrict__ x,
                                                                const float* __restrict__ phi,
                                                                float* __restrict__ part, int64_t R, int64_t K,
                                                                int nK, int64_t KC, bool phi_vec) {
  __shared__ float lds[4 * RT * kPart];
  const int64_t r0 = (int64_t)blockIdx.x * RT;
  const int kc = blockIdx.y;
  float acc[RT * kPart];
#pragma unroll
  for (int i = 0; i < RT * kPart; ++i) acc[i] = 0.f;
  const int64_t kbeg = (int64_t)kc * KC;
  const int64_t kend = kbeg + KC < K ? kbeg + KC : K;
  for (int64_t k = kbeg + threadIdx.x; k < kend; k += kThreads) {
    float ph[kOut];
    load_phi_row(phi, k, phi_vec, ph);
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      if (r0 + r < R) {
        const float xv = to_f32(x[(r0 + r) * K + k]);
        acc[r * kPart + kOut] += xv * xv;
#pragma unroll
        for (int j = 0; j < kOut; ++j) acc[r * kPart + j] += xv * ph[j];
      }
    }
  }
  block_sum<RT * kPart>(acc, lds);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      if (r0 + r < R) {
        float* pp = part + ((r0 + r) * nK + kc) * kPart;
#pragma unroll
        for (int j = 0; j < kPart; ++j) pp[j] = acc[r * kPart + j];
      }
    }
  }
}

struct DynParams {
  const float* bias_pre;   // [4]
  const float* bias_post;  // [4]
  const float* bias_res;   // [16]
  const float* alpha_pre;  // [1]
  const float* alpha_post; // [1]
  const float* alpha_res;  // [1]
};

__device__ __forceinline__ float sigmoidf(float v) { return 1.f / (1.f + expf(-v)); }

// scaled[j] = inv_rms * alpha_g * raw[j] + bias[j]
__device__ __forceinline__ void dyn_scaled(const DynParams& P, const float (&raw)[kOut], float inv_rms,
                                           float (&s)[kOut]) {
  const float ap = *P.alpha_pre, aq = *P.alpha_post, ar = *P.alpha_res;
#pragma unroll
  for (int j = 0; j < 4; ++j) s[j] = inv_rms * ap * raw[j] + P.bias_pre[j];
#pragma unroll
  for (int j = 0; j < 4; ++j) s[4 + j] = inv_rms * aq * raw[4 + j] + P.bias_post[j];
#pragma unroll
  for (int j = 0; j < 16; ++j) s[8 + j] = inv_rms * ar * raw[8 + j] + P.bias_res[j];
}

// One wave per row.  Lane l sums the partial records l, l+64, l+128, ... (25
// floats each) in chunk order, the wave then adds the 64 lane sums with a
// fixed butterfly, and lane 0 runs the epilogue.  Keeping 64 independent load
// streams per row instead of one serial chain matters: R is the batch (4 at
// dim 4096) and this kernel sits between two full passes over H.
template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_finalize_kernel(const float* __restrict__ part, int nK, int64_t R,
                                                                 int64_t K, DynParams P, OutRow o_pre,
                                                                 OutRow o_post, OutRow o_res,
                                                                 float* __restrict__ aux, int iters, float eps) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  if (r >= R) return;
  float acc[kPart];
#pragma unroll
  for (int j = 0; j < kPart; ++j) acc[j] = 0.f;
  for (int k = lane; k < nK; k += 64) {
    const float* p = part + (r * nK + k) * kPart;
#pragma unroll
    for (int j = 0; j < kPart; ++j) acc[j] += p[j];
  }
#pragma unroll
  for (int j = 0; j < kPart; ++j) acc[j] = wave_sum(acc[j]);
  if (lane != 0) return;
  float raw[kOut];
#pragma unroll
  for (int j = 0; j < kOut; ++j) raw[j] = acc[j];
  const float inv_rms = 1.f / sqrtf(acc[kOut] / (float)K + eps);
  float s[kOut];
  dyn_scaled(P, raw, inv_rms, s);
  // Eq. 17: H_pre = sigmoid / (sum + eps)
  float sg[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sg[j] = sigmoidf(s[j]);
  const float den = sg[0] + sg[1] + sg[2] + sg[3] + eps;
#pragma unroll
  for (int j = 0; j < 4; ++j) o_pre.p[r * o_pre.stride + j] = sg[j] / den;
  // Eq. 18: H_post = 2 sigmoid
#pragma unroll
  for (int j = 0; j < 4; ++j) o_post.p[r * o_post.stride + j] = 2.f * sigmoidf(s[4 + j]);
  // Eq. 19: H_res = Sinkhorn(|s_res| + eps)
  float m[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) m[j] = s[8 + j];
  sk_forward(m, iters, eps);
#pragma unroll
  for (int j = 0; j < 16; ++j) o_res.p[r * o_res.stride + j] = m[j];
  if (aux) {
#pragma unroll
    for (int j = 0; j < kOut; ++j) aux[r * kPart + j] = raw[j];
    aux[r * kPart + kOut] = inv_rms;
  }
}

// Per-row backward record rowbuf[r][0:52]:
//   [0:24]  grad_raw  = g_scaled * inv_rms * alpha_g
//   [24]    coef      : grad_x += coef * x  (rms path)
//   [25:49] g_scaled  (-> grad_bias)
//   [49:52] per-group sum g_scaled * inv_rms * raw (-> grad_alpha)
// Follows reference src/mhc/ops.py:138-216 with the Sinkhorn part of
// _backward.py:29-262 (sgn(0) = 0).
template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_bwd_rows_kernel(const float* __restrict__ aux, DynParams P,
                                                                 InRow h_pre, InRow g_pre, InRow g_post,
                                                                 InRow g_res, float* __restrict__ rowbuf,
                                                                 int64_t R, int64_t K, int iters, float eps) {
  const int64_t r = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (r >= R) return;
  float raw[kOut];
#pragma unroll
  for (int j = 0; j < kOut; ++j) raw[j] = aux[r * kPart + j];
  const float inv_rms = aux[r * kPart + kOut];
  float s[kOut];
  dyn_scaled(P, raw, inv_rms, s);
  float gs[kOut];
  // H_res: Sinkhorn backward w.r.t. scaled_res
  {
    float m[16], d[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      m[j] = s[8 + j];
      d[j] = g_res.p ? g_res.p[r * g_res.stride + j] : 0.f;
    }
    sk_backward<10>(m, d, iters, eps);
#pragma unroll
    for (int j = 0; j < 16; ++j) gs[8 + j] = d[j];
  }
  // H_post = 2 sigmoid: g * 2 sig (1 - sig)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float sg = sigmoidf(s[4 + j]);
    const float g = g_post.p ? g_post.p[r * g_post.stride + j] : 0.f;
    gs[4 + j] = g * 2.f * sg * (1.f - sg);
  }
  // H_pre = sig / (sum sig + eps)
  {
    float sg[4], g[4], hp[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sg[j] = sigmoidf(s[j]);
      g[j] = g_pre.p ? g_pre.p[r * g_pre.stride + j] : 0.f;
      hp[j] = h_pre.p[r * h_pre.stride + j];
    }
    const float den = sg[0] + sg[1] + sg[2] + sg[3] + eps;
    const float dot = g[0] * hp[0] + g[1] * hp[1] + g[2] * hp[2] + g[3] * hp[3];
#pragma unroll
    for (int j = 0; j < 4; ++j) gs[j] = (g[j] - dot) / den * sg[j] * (1.f - sg[j]);
  }
  const float al[3] = {*P.alpha_pre, *P.alpha_post, *P.alpha_res};
  float* rb = rowbuf + r * kRow;
  float ga[3] = {0.f, 0.f, 0.f};
  float g_inv = 0.f;
#pragma unroll
  for (int j = 0; j < kOut; ++j) {
    const int grp = j < 4 ? 0 : (j < 8 ? 1 : 2);
    rb[j] = gs[j] * inv_rms * al[grp];
    rb[25 + j] = gs[j];
    ga[grp] += gs[j] * inv_rms * raw[j];
    g_inv += gs[j] * al[grp] * raw[j];
  }
  // inv_rms = 1/rms, rms = sqrt(sum x^2 / K + eps): d rms / d x = x / (K rms)
  const float grad_rms = g_inv * (-inv_rms * inv_rms);
  rb[24] = grad_rms * inv_rms / (float)K;
#pragma unroll
  for (int g = 0; g < 3; ++g) rb[49 + g] = ga[g];
}

// Thread per k.  grad_x (f32) rows have stride K.
template <typename TX>
__global__ __launch_bounds__(kThreads) void dynw_bwd_wide_kernel(const TX* __restrict__ x,
                                                                 const float* __restrict__ phi,
                                                                 const float* __restrict__ rowbuf,
                                                                 float* __restrict__ gx, float* __restrict__ gphi,
                                                                 int64_t R, int64_t K, bool phi_vec) {
  const int64_t k = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (k >= K) return;
  float ph[kOut], gp[kOut];
  load_phi_row(phi, k, phi_vec, ph);
#pragma unroll
  for (int j = 0; j < kOut; ++j) gp[j] = 0.f;
  for (int64_t r = 0; r < R; ++r) {
    const float* rb = rowbuf + r * kRow;
    const float xv = to_f32(x[r * K + k]);
    float v = rb[24] * xv;
#pragma unroll
    for (int j = 0; j < kOut; ++j) {
      v += rb[j] * ph[j];
      gp[j] += xv * rb[j];
    }
    if (gx) gx[r * K + k] = v;
  }
  if (gphi) {
    float* o = gphi + k * kOut;
#pragma unroll
    for (int j = 0; j < kOut; ++j) o[j] = gp[j];
  }
}

// Single workgroup: grad_bias[24], grad_alpha[3] summed over rows in a fixed order.
template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_bwd_sum_kernel(const float* __restrict__ rowbuf, int64_t R,
                                                                float* __restrict__ gbias,
                                                                float* __restrict__ galpha) {
  __shared__ float lds[4 * 27];
  float acc[27];
#pragma unroll
  for (int i = 0; i < 27; ++i) acc[i] = 0.f;
  for (int64_t r = threadIdx.x; r < R; r += kThreads) {
    const float* rb = rowbuf + r * kRow;
#pragma unroll
    for (int i = 0; i < 27; ++i) acc[i] += rb[25 + i];
  }
  block_sum<27>(acc, lds);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < kOut; ++j) if (gbias) gbias[j] = acc[j];
#pragma unroll
    for (int g = 0; g < 3; ++g) if (galpha) galpha[g] = acc[24 + g];
  }
}

// ---------------------------------------------------------------------------
// Sequence mean-pool, module.py:123: x[b, c] = (1/S) sum_s H[b, s, c] over the
// flattened [S, K = 4D] view (c = n*D + d), in two launches.
//
// colsum_kernel: grid (column chunks, S chunks, batch).  A workgroup owns
//   256*W columns (one 16-byte vector per lane: the workgroup reads 4 KiB of a
//   row contiguously) and SC consecutive rows, which it walks with UN rows in
//   flight per lane; each lane sums its own W columns, so no cross-lane step
//   is needed, and the fp32 sums of the chunk go to colpart[b][sc][c].
//   Splitting S gives enough workgroups at B = 1, but not too many: on MI355X
//   this read peaks (80% of 8 TB/s) with about 1.5 workgroups x 4 rows in
//   flight per CU; twice that loses 10%.
// colsum_reduce_kernel: one thread per column sums the S-chunk partials in
//   chunk order, scales by 1/S and writes x; with PROJ it also forms the 25
//   projection partials of its 256 columns (x . phi[c,:] and x^2), so the
//   dynamic-weight projection needs no extra pass over x.
// ---------------------------------------------------------------------------
template <typename T, int W, int UN>
__global__ __launch_bounds__(kThreads) void colsum_kernel(const T* __restrict__ H, float* __restrict__ colpart,
                                                          int64_t S, int64_t K, int64_t SC, int nS, int64_t b0) {
  const int64_t b = b0 + blockIdx.z;
  const int sc = blockIdx.y;
  const int64_t col = (int64_t)blockIdx.x * (kThreads * W) + (int64_t)threadIdx.x * W;
  if (col >= K) return;
  const int64_t sbeg = (int64_t)sc * SC;
  const int64_t send = sbeg + SC < S ? sbeg + SC : S;
  float acc[W];
#pragma unroll
  for (int e = 0; e < W; ++e) acc[e] = 0.f;
  const T* p = H + b * S * K + col;
  int64_t s = sbeg;
  for (; s + (UN - 1) < send; s += UN) {
    float v[UN][W];
#pragma unroll
    for (int u = 0; u < UN; ++u) ld<T, W>(p + (s + u) * K, v[u]);
#pragma unroll
    for (int u = 0; u < UN; ++u)
#pragma unroll
      for (int e = 0; e < W; ++e) acc[e] += v[u][e];
  }
  for (; s < send; ++s) {
    float v[W];
    ld<T, W>(p + s * K, v);
#pragma unroll
    for (int e = 0; e < W; ++e) acc[e] += v[e];
  }
  st<float, W>(colpart + ((b * nS + sc) * K + col), acc);
}

template <bool PROJ>
__global__ __launch_bounds__(kThreads) void colsum_reduce_kernel(const float* __restrict__ colpart,
                                                                 float* __restrict__ x,
                                                                 const float* __restrict__ phi,
                                                                 float* __restrict__ projpart, int64_t K, int nS,
                                                                 float inv_S, int64_t b0, bool phi_vec) {
  __shared__ float red[4 * kPart];
  const int64_t b = b0 + blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float pv[kPart];
#pragma unroll
  for (int j = 0; j < kPart; ++j) pv[j] = 0.f;
  if (c < K) {
    const float* p = colpart + b * nS * K + c;
    float v = 0.f;
#pragma unroll 8
    for (int k = 0; k < nS; ++k) v += p[(int64_t)k * K];
    v *= inv_S;
    x[b * K + c] = v;
    if constexpr (PROJ) {
      float ph[kOut];
      load_phi_row(phi, c, phi_vec, ph);
#pragma unroll
      for (int j = 0; j < kOut; ++j) pv[j] = v * ph[j];
      pv[kOut] = v * v;
    }
  }
  if constexpr (PROJ) {
    block_sum<kPart>(pv, red);
    if (threadIdx.x == 0) {
      float* pp = projpart + (b * gridDim.x + blockIdx.x) * kPart;
#pragma unroll
      for (int j = 0; j < kPart; ++j) pp[j] = pv[j];
    }
  }
}

// Launch plan of the two mean-pool kernels; depends only on the shape, so
// workspace sizes can be queried without a device.
struct PoolPlan {
  int W;         // elements per lane (16 bytes, or 1 on the unaligned path)
  int64_t ncc;   // column chunks of 256*W
  int64_t SC;    // rows per S chunk
  int nS;        // S chunks
  int64_t nrc;   // column chunks of the reduce kernel (256 columns)
};

constexpr int kPoolWG = 384;  // target colsum workgroups: 1.5 per CU on MI355X

__host__ inline PoolPlan pool_plan(int64_t B, int64_t S, int64_t K, int W) {
  PoolPlan p;
  p.W = W;
  p.ncc = (K + kThreads * W - 1) / (kThreads * W);
  if (p.ncc < 1) p.ncc = 1;
  const int64_t per = p.ncc * (B > 0 ? B : 1);
  int64_t ns = (kPoolWG + per - 1) / per;
  if (ns < 1) ns = 1;
  int64_t sc = S > 0 ? (S + ns - 1) / ns : 1;
  p.SC = sc;
  p.nS = S > 0 ? (int)((S + sc - 1) / sc) : 1;
  p.nrc = (K + kThreads - 1) / kThreads;
  if (p.nrc < 1) p.nrc = 1;
  return p;
}

}  // namespace mhc
