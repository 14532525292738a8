// Register-resident Sinkhorn-Knopp on one 4x4 matrix per lane.
//
// Forward (reference src/mhc/_torch_baseline.py:27-35, _kernels.py:75-112):
//   P = |M| + eps;  repeat iters: P /= (rowsum(P) + eps); P /= (colsum(P) + eps)
// Row and column sums are accumulated left to right as in the reference
// (sk_forward carries the same iteration as two reciprocal scaling vectors, below).
// A division P/r is computed as P * rcp(r): one v_rcp_f32 per row/column
// instead of four IEEE divides; the result stays within a few ulp of the
// divided form (checked against an fp64 oracle by the parity tests).
//
// Backward (reference src/mhc/_backward.py:29-262): reverse mode through every
// row/column normalisation, y = x/s  =>  dx = (dy - <dy, y>) / s, and finally
// dM = dP0 * sgn(M) with sgn(0) = 0 as in torch autograd of |M| (the reference
// Triton kernel uses +1 at 0; the pure-PyTorch path, the parity target, uses 0).
//
// The reference recomputes the forward from M for every iteration it
// differentiates (T(T-1)/2 = 190 extra rounds at T = 20).  Here the forward is
// checkpointed every L = ceil(T / NCK) rounds in registers and each state is
// recomputed from the nearest checkpoint; the recomputed states are
// bit-identical to the ones a full recompute produces (same instruction
// sequence), at 48 instead of 210 rounds for T = 20 with NCK = 10.  The ten
// checkpoints hold 160 registers (234 VGPRs, 2 waves per SIMD); at 2^20
// matrices that runs in 163 us against 191 us with NCK = 5 (66 rounds, 154
// VGPRs, 3 waves per SIMD) -- the kernel is VALU-bound, so fewer rounds win.
#pragma once

#include "common.hpp"

namespace mhc {

__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }

// One Sinkhorn round (row normalisation then column normalisation), in place.
__device__ __forceinline__ void sk_round(float (&m)[16], float eps) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float q = fast_rcp(m[4 * i] + m[4 * i + 1] + m[4 * i + 2] + m[4 * i + 3] + eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) m[4 * i + j] *= q;
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float q = fast_rcp(m[j] + m[4 + j] + m[8 + j] + m[12 + j] + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) m[4 * i + j] *= q;
  }
}

// P0 = |M| + eps.
__device__ __forceinline__ void sk_init(float (&m)[16], float eps) {
#pragma unroll
  for (int k = 0; k < 16; ++k) m[k] = __builtin_fabsf(m[k]) + eps;
}

// The forward kernel's iteration in scaling-vector form: after any number of
// rounds P = diag(u) P0 diag(v), and the kernel carries w = 1/u and z = 1/v.
// A row normalisation u_i <- u_i / (u_i (P0 v)_i + eps) is then
//   w_i <- (P0 v)_i + eps w_i          (one mul + 3 FMAs for the dot, one FMA)
// with v = rcp(z), and a column normalisation likewise updates z from
// u = rcp(w); P is formed once at the end.  That is the same sequence of
// normalisations at 40 VALU + 8 v_rcp per round, against 64 + 8 for
// sk_round's explicit update (at 2^20 matrices 41 us against 52 us; 48 + 8
// when carrying u and v themselves), with a normwise error against an fp64
// evaluation of the explicit form of 1.7e-7 (2.2e-7 for the explicit fp32
// update).  The backward keeps sk_round for its recomputed states.
__device__ __forceinline__ void sk_forward(float (&m)[16], int iters, float eps) {
  sk_init(m, eps);
  float w[4] = {1.f, 1.f, 1.f, 1.f}, z[4] = {1.f, 1.f, 1.f, 1.f};
  for (int t = 0; t < iters; ++t) {
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = fast_rcp(z[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float dot = m[4 * i] * v[0] + m[4 * i + 1] * v[1] + m[4 * i + 2] * v[2] + m[4 * i + 3] * v[3];
      w[i] = __builtin_fmaf(eps, w[i], dot);
    }
    float u[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) u[i] = fast_rcp(w[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dot = u[0] * m[j] + u[1] * m[4 + j] + u[2] * m[8 + j] + u[3] * m[12 + j];
      z[j] = __builtin_fmaf(eps, z[j], dot);
    }
  }
  float u[4], v[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    u[k] = fast_rcp(w[k]);
    v[k] = fast_rcp(z[k]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) m[4 * i + j] = u[i] * m[4 * i + j] * v[j];
}

// Given the state m entering a round and the gradient d w.r.t. the state
// leaving it, replace d by the gradient w.r.t. m.
__device__ __forceinline__ void sk_round_backward(const float (&m)[16], float (&d)[16], float eps) {
  float r[4], mr[16], c[4], mc[16];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = fast_rcp(m[4 * i] + m[4 * i + 1] + m[4 * i + 2] + m[4 * i + 3] + eps);
#pragma unroll
    for (int j = 0; j < 4; ++j) mr[4 * i + j] = m[4 * i + j] * r[i];
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c[j] = fast_rcp(mr[j] + mr[4 + j] + mr[8 + j] + mr[12 + j] + eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) mc[4 * i + j] = mr[4 * i + j] * c[j];
  }
  // Column normalisation: dmr[:,j] = (d[:,j] - <d[:,j], mc[:,j]>) / colsum_j,
  // evaluated as d c - <.,.> c: one FMA per element and one multiply per
  // column instead of a subtract and a multiply per element.
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float dot = d[j] * mc[j] + d[4 + j] * mc[4 + j] + d[8 + j] * mc[8 + j] + d[12 + j] * mc[12 + j];
    const float dc = dot * c[j];
#pragma unroll
    for (int i = 0; i < 4; ++i) d[4 * i + j] = __builtin_fmaf(d[4 * i + j], c[j], -dc);
  }
  // Row normalisation: dm[i,:] = (dmr[i,:] - <dmr[i,:], mr[i,:]>) / rowsum_i.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float dot = d[4 * i] * mr[4 * i] + d[4 * i + 1] * mr[4 * i + 1] + d[4 * i + 2] * mr[4 * i + 2] +
                      d[4 * i + 3] * mr[4 * i + 3];
    const float dr = dot * r[i];
#pragma unroll
    for (int j = 0; j < 4; ++j) d[4 * i + j] = __builtin_fmaf(d[4 * i + j], r[i], -dr);
  }
}

// Gradient of Sinkhorn(M) w.r.t. M.  On entry `mat` holds M and `d` holds the
// gradient w.r.t. the output P; on exit `d` holds dM.
template <int NCK = 10>
__device__ __forceinline__ void sk_backward(const float (&mat)[16], float (&d)[16], int iters, float eps) {
  float m[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) m[k] = mat[k];
  sk_init(m, eps);
  const int L = (iters + NCK - 1) / NCK;  // rounds per segment
  float ck[NCK][16];
#pragma unroll
  for (int k = 0; k < NCK; ++k) {
#pragma unroll
    for (int e = 0; e < 16; ++e) ck[k][e] = m[e];
    if (k + 1 < NCK) {
      const int t1 = min(iters, (k + 1) * L);
      for (int t = k * L; t < t1; ++t) sk_round(m, eps);
    }
  }
#pragma unroll
  for (int k = NCK - 1; k >= 0; --k) {
    const int t0 = k * L;
    const int t1 = min(iters, t0 + L);
    for (int t = t1 - 1; t >= t0; --t) {
      float s[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) s[e] = ck[k][e];
      for (int u = t0; u < t; ++u) sk_round(s, eps);
      sk_round_backward(s, d, eps);
    }
  }
  // d|M|/dM = sgn(M), sgn(0) = 0.
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float sg = mat[e] > 0.f ? 1.f : (mat[e] < 0.f ? -1.f : 0.f);
    d[e] *= sg;
  }
}

// The same gradient for iters <= TMAX from the scaling vectors of every round,
// kept in registers instead of recomputed from checkpoints.  After t rounds
// P = diag(u_t) P0 diag(v_t), with u_0 = v_0 = 1; the forward runs as in
// sk_forward (carrying w = 1/u and z = 1/v) and keeps u_t and v_t, 8 floats
// per round.  Round t maps u_t to u_{t+1} = r u_t (r = 1 / (rowsum + eps)) and
// then v_t to v_{t+1} = c v_t (c = 1 / (colsum + eps)).  The adjoint is
// carried in scaled coordinates: the gradient dP of a state P0 u v^T is held
// as g = dP * u v^T (elementwise).  The column normalisation backward,
// dA_ij = c_j (dB_ij - sum_k dB_kj B_kj), then reads
//   g_ij <- g_ij - u_{t+1},i v_{t+1},j sum_k g_kj P0_kj,
// because B = P0 u_{t+1} v_{t+1}^T and c_j v_t,j = v_{t+1},j; and the row
// normalisation backward, dP_ij = r_i (dA_ij - sum_l dA_il A_il),
//   g_ij <- g_ij - v_t,j u_{t+1},i sum_l g_il P0_il,
// because A = P0 u_{t+1} v_t^T and r_i u_t,i = u_{t+1},i.  A round is two
// 16-term dot passes over g * P0 and two FMA updates, 72 VALU and no v_rcp
// (the explicit form of sk_round_backward on the scaled state took about
// 128 + 8 v_rcp); the forward is 40 VALU + 8 v_rcp per round.  g starts as
// dP_T * u_T v_T^T and ends as dP0 (u_0 = v_0 = 1).
template <int TMAX>
__device__ __forceinline__ void sk_backward_scaled(const float (&mat)[16], float (&d)[16], int iters, float eps) {
  float p0[16];
  uint32_t neg = 0u, zero = 0u;  // sgn(M) as two bit masks, so that M need not stay live
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    p0[k] = __builtin_fabsf(mat[k]) + eps;
    neg |= (mat[k] < 0.f ? 1u : 0u) << k;
    zero |= (mat[k] == 0.f ? 1u : 0u) << k;
  }
  float U[TMAX + 1][4], V[TMAX + 1][4];
#pragma unroll
  for (int k = 0; k < 4; ++k) U[0][k] = V[0][k] = 1.f;
  {
    float w[4] = {1.f, 1.f, 1.f, 1.f}, z[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int t = 0; t < TMAX; ++t) {
      if (t < iters) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float dot = p0[4 * i] * V[t][0] + p0[4 * i + 1] * V[t][1] + p0[4 * i + 2] * V[t][2] +
                            p0[4 * i + 3] * V[t][3];
          w[i] = __builtin_fmaf(eps, w[i], dot);
          U[t + 1][i] = fast_rcp(w[i]);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float dot = U[t + 1][0] * p0[j] + U[t + 1][1] * p0[4 + j] + U[t + 1][2] * p0[8 + j] +
                            U[t + 1][3] * p0[12 + j];
          z[j] = __builtin_fmaf(eps, z[j], dot);
          V[t + 1][j] = fast_rcp(z[j]);
        }
      }
    }
  }
#pragma unroll
  for (int t = TMAX - 1; t >= 0; --t) {
    if (t == iters - 1) {  // the last round: g = dP_T * u_T v_T^T
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) d[4 * i + j] *= U[t + 1][i] * V[t + 1][j];
    }
    if (t < iters) {
      // column normalisation of round t
      float e[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        e[j] = (d[j] * p0[j] + d[4 + j] * p0[4 + j] + d[8 + j] * p0[8 + j] + d[12 + j] * p0[12 + j]) * V[t + 1][j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) d[4 * i + j] = __builtin_fmaf(-U[t + 1][i], e[j], d[4 * i + j]);
      // row normalisation of round t
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float f = (d[4 * i] * p0[4 * i] + d[4 * i + 1] * p0[4 * i + 1] + d[4 * i + 2] * p0[4 * i + 2] +
                         d[4 * i + 3] * p0[4 * i + 3]) *
                        U[t + 1][i];
#pragma unroll
        for (int j = 0; j < 4; ++j) d[4 * i + j] = __builtin_fmaf(-V[t][j], f, d[4 * i + j]);
      }
    }
  }
  // d|M|/dM = sgn(M), sgn(0) = 0.
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float sg = (zero >> e) & 1u ? 0.f : ((neg >> e) & 1u ? -1.f : 1.f);
    d[e] *= sg;
  }
}

// The scaled-coordinate gradient for more rounds than fit in registers:
// NSEG segments of up to TSEG rounds.  The forward keeps only the carried
// reciprocal vectors (w, z) at the start of each segment; the backward then
// walks the segments from the last, recomputes the segment's u and v from its
// checkpoint (the same rcp of the same carried values, so bit-identical to the
// forward's) and runs sk_backward_scaled's round backward over them.  Every
// round is recomputed once, against several times for the explicit-state
// checkpoints of sk_backward.  Requires iters <= TSEG * NSEG.
template <int TSEG, int NSEG>
__device__ __forceinline__ void sk_backward_segmented(const float (&mat)[16], float (&d)[16], int iters, float eps) {
  float p0[16];
  uint32_t neg = 0u, zero = 0u;
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    p0[k] = __builtin_fabsf(mat[k]) + eps;
    neg |= (mat[k] < 0.f ? 1u : 0u) << k;
    zero |= (mat[k] == 0.f ? 1u : 0u) << k;
  }
  // one round of the carried iteration: w from v, u = rcp(w), z from u, v = rcp(z)
  auto sk_step = [&](float (&w)[4], float (&z)[4], const float (&v)[4], float (&u1)[4], float (&v1)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float dot = p0[4 * i] * v[0] + p0[4 * i + 1] * v[1] + p0[4 * i + 2] * v[2] + p0[4 * i + 3] * v[3];
      w[i] = __builtin_fmaf(eps, w[i], dot);
      u1[i] = fast_rcp(w[i]);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float dot = u1[0] * p0[j] + u1[1] * p0[4 + j] + u1[2] * p0[8 + j] + u1[3] * p0[12 + j];
      z[j] = __builtin_fmaf(eps, z[j], dot);
      v1[j] = fast_rcp(z[j]);
    }
  };
  float cw[NSEG][4], cz[NSEG][4];
  {
    float w[4] = {1.f, 1.f, 1.f, 1.f}, z[4] = {1.f, 1.f, 1.f, 1.f}, v[4] = {1.f, 1.f, 1.f, 1.f};
#pragma unroll
    for (int k = 0; k < NSEG; ++k) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cw[k][q] = w[q];
        cz[k][q] = z[q];
      }
      const int tend = iters < (k + 1) * TSEG ? iters : (k + 1) * TSEG;
      for (int t = k * TSEG; t < tend; ++t) {
        float u1[4], v1[4];
        sk_step(w, z, v, u1, v1);
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = v1[q];
      }
    }
    // g = dP_T * u_T v_T^T
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float u = fast_rcp(w[i]);
#pragma unroll
      for (int j = 0; j < 4; ++j) d[4 * i + j] *= u * fast_rcp(z[j]);
    }
  }
  for (int k = (iters + TSEG - 1) / TSEG - 1; k >= 0; --k) {
    const int t0 = k * TSEG;
    float U[TSEG + 1][4], V[TSEG + 1][4], w[4], z[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = z[q] = 1.f;
#pragma unroll
    for (int c = 0; c < NSEG; ++c)
      if (c == k) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          w[q] = cw[c][q];
          z[q] = cz[c][q];
        }
      }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      U[0][q] = fast_rcp(w[q]);
      V[0][q] = fast_rcp(z[q]);
    }
#pragma unroll
    for (int tt = 0; tt < TSEG; ++tt)
      if (t0 + tt < iters) sk_step(w, z, V[tt], U[tt + 1], V[tt + 1]);
#pragma unroll
    for (int tt = TSEG - 1; tt >= 0; --tt) {
      if (t0 + tt < iters) {
        float e[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          e[j] = (d[j] * p0[j] + d[4 + j] * p0[4 + j] + d[8 + j] * p0[8 + j] + d[12 + j] * p0[12 + j]) * V[tt + 1][j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j) d[4 * i + j] = __builtin_fmaf(-U[tt + 1][i], e[j], d[4 * i + j]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float f = (d[4 * i] * p0[4 * i] + d[4 * i + 1] * p0[4 * i + 1] + d[4 * i + 2] * p0[4 * i + 2] +
                           d[4 * i + 3] * p0[4 * i + 3]) *
                          U[tt + 1][i];
#pragma unroll
          for (int j = 0; j < 4; ++j) d[4 * i + j] = __builtin_fmaf(-V[tt][j], f, d[4 * i + j]);
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float sg = (zero >> e) & 1u ? 0.f : ((neg >> e) & 1u ? -1.f : 1.f);
    d[e] *= sg;
  }
}

// ---------------------------------------------------------------------------
// 16-lane form, for the latency-bound per-row kernels (a handful of matrices,
// one per batch row): one matrix is spread over 16 consecutive lanes, lane
// e = 4 i + j holding P[i][j].  Row sums are two quad-permute DPP adds, column
// sums two row-rotate DPP adds (rotate by 8, then by 4, within the 16 lanes),
// so a round is about 10 dependent instructions instead of about 70 on one
// lane.  Both trees add the same pairs in every lane, so all lanes of a row
// (column) see bit-identical sums.  All 16 lanes of a group must be active.
// The serial one-matrix-per-lane form above stays the throughput choice for
// large batches of matrices (fewer instructions per matrix).
// ---------------------------------------------------------------------------
// (dpp, sum_row16, sum_col16 and sum_all16 are in common.hpp.)
__device__ __forceinline__ float sk16_round(float m, float eps) {
  m *= fast_rcp(sum_row16(m) + eps);
  return m * fast_rcp(sum_col16(m) + eps);
}

__device__ __forceinline__ float sk16_forward(float m, int iters, float eps) {
  m = __builtin_fabsf(m) + eps;
  for (int t = 0; t < iters; ++t) m = sk16_round(m, eps);
  return m;
}

// Gradient w.r.t. the state m entering a round, given the gradient d w.r.t.
// the state leaving it (same normalisation backward as sk_round_backward).
__device__ __forceinline__ float sk16_round_backward(float m, float d, float eps) {
  const float r = fast_rcp(sum_row16(m) + eps);
  const float mr = m * r;
  const float c = fast_rcp(sum_col16(mr) + eps);
  const float mc = mr * c;
  d = (d - sum_col16(d * mc)) * c;
  return (d - sum_row16(d * mr)) * r;
}

// sk16_backward for a compile-time iteration count: every forward state stays
// in a register (one per round per lane) and both sweeps are unrolled, so a
// round costs only its dependent VALU / DPP chain.
template <int T>
__device__ __forceinline__ float sk16_backward_fixed(float mat, float d, float eps) {
  float st[T > 0 ? T : 1];
  float m = __builtin_fabsf(mat) + eps;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    st[t] = m;
    m = sk16_round(m, eps);
  }
#pragma unroll
  for (int t = T - 1; t >= 0; --t) d = sk16_round_backward(st[t], d, eps);
  const float sg = mat > 0.f ? 1.f : (mat < 0.f ? -1.f : 0.f);
  return d * sg;
}

// dM for one matrix in 16-lane form.  The forward states are kept in `slot`
// (this lane's LDS slots, `stride` floats apart): every state when
// iters <= NSLOT, otherwise every L-th state with the rest recomputed from the
// nearest kept one (the recomputed states are bit-identical to the forward's).
template <int NSLOT>
__device__ __forceinline__ float sk16_backward(float mat, float d, int iters, float eps, float* slot, int stride) {
  const int L = iters <= NSLOT ? 1 : (iters + NSLOT - 1) / NSLOT;
  float m = __builtin_fabsf(mat) + eps;
  for (int t = 0; t < iters; ++t) {
    if (t % L == 0) slot[(t / L) * stride] = m;
    m = sk16_round(m, eps);
  }
  for (int t = iters - 1; t >= 0; --t) {
    const int k = t / L;
    float st = slot[k * stride];
    for (int u = k * L; u < t; ++u) st = sk16_round(st, eps);
    d = sk16_round_backward(st, d, eps);
  }
  // d|M|/dM = sgn(M), sgn(0) = 0.
  const float sg = mat > 0.f ? 1.f : (mat < 0.f ? -1.f : 0.f);
  return d * sg;
}

}  // namespace mhc
