// HBM-streaming kernels over the (B, S, 4, D) stream tensor.
//
// Work decomposition (all kernels here): grid.y = batch (so the 4-24 mixing
// weights of a batch are wave-uniform scalar loads), grid.x = workgroups per
// batch.  The per-batch index space is S * D/W "items"; an item is W
// consecutive elements of one token row (W = 16 bytes worth, 4 fp32 or 8
// bf16/fp16; W = 1 on the unaligned / ragged-D path) across all 4 streams.
// Consecutive lanes take consecutive items, so each wave access is one
// contiguous 1 KiB span per stream row.  A workgroup processes tiles of
// 256 * U items (U = 1: a lane keeps 4-5 16-byte loads in flight; the
// reduction-only pass uses U = 2).  Kernels that reduce over (s, d) stride over
// tiles and write one partial vector per workgroup; reduce_split_kernel then
// sums them in a fixed order (deterministic).
#pragma once

#include "common.hpp"

namespace mhc {

// ---------------------------------------------------------------------------
// Launch shape of the streaming kernels, measured on MI355X (gfx950: 256 CUs,
// 160 KiB LDS per CU).  HBM throughput of these kernels peaks with roughly
// 24-40 KiB of loads in flight per CU; more resident workgroups lower it (the
// closure forward, 5 loads per lane, runs at 73% of 8 TB/s with 8 workgroups
// per CU and at 75-77% with 2-3; the closure backward at 69% and 74%).  The kernels use almost no LDS, so the cap is set
// by reserving dynamic LDS at launch: at most `wg_per_cu` workgroups fit on a
// CU.  Streamed tensors are read and written with the streaming (nt) cache
// policy (NT bit 0: loads, bit 1: stores).  Through buffer spans (Span) nt
// loads and stores lift the closure forward from 76% to 79-81% of 8 TB/s; on
// 64-bit global addressing only the nt stores helped (3-6%).
// ---------------------------------------------------------------------------
constexpr size_t kLdsPerCu = 160 * 1024;

inline size_t occupancy_lds(int wg_per_cu) {
  return wg_per_cu <= 0 ? 0 : (kLdsPerCu / (size_t)wg_per_cu - 1024) & ~(size_t)255;
}

constexpr int kNt = 3;

// Load order inside a tile.  The forward kernels load every vector of the
// tile into raw fragments, keep the compiler from starting to unpack before
// the last load is issued (scheduling barrier), then unpack: +2-5% (the
// closure forward 74% -> 77% of 8 TB/s).  The backward kernels, which carry
// 9-13 loads per item, unpack each vector as it is loaded (ld<>): held back
// that way they lose 2-5%.
__device__ __forceinline__ void loads_issued() { __builtin_amdgcn_sched_barrier(0); }

// Per-batch fp32 weight rows: element n of batch b is p[b * stride + n].
struct WRow {
  const float* p;
  int64_t stride;
};

struct Geom {
  int64_t S, D;   // sequence, per-stream dim
  uint32_t nch;   // D / W
  uint32_t items; // S * nch
  uint32_t ntiles;
  int64_t b0;     // first batch of this launch
};

template <int W, int U>
__host__ inline Geom make_geom(int64_t S, int64_t D, int64_t b0) {
  Geom g;
  g.S = S;
  g.D = D;
  g.nch = (uint32_t)(D / W);
  g.items = (uint32_t)(S * (D / W));
  g.ntiles = (g.items + kThreads * U - 1) / (kThreads * U);
  g.b0 = b0;
  return g;
}

__device__ __forceinline__ void load_w4(WRow w, int64_t b, float (&v)[4]) {
#pragma unroll
  for (int n = 0; n < 4; ++n) v[n] = w.p[b * w.stride + n];
}

__device__ __forceinline__ void load_w16(WRow w, int64_t b, float (&v)[16]) {
#pragma unroll
  for (int n = 0; n < 16; ++n) v[n] = w.p[b * w.stride + n];
}

// ---------------------------------------------------------------------------
// Forward mixing from H.
//   BI:   bi[s,:]        = sum_n pre[n] H[s,n,:]
//   RES:  out[s,n,:]     = sum_m res[n,m] H[s,m,:]            (+ ADD_BO)
//   ADD_BO: out[s,n,:]  += post[n] bo[s,:]
// Used for fused_stream_mix (BI + RES), the layer's branch_input pass (BI)
// and the layer closure (RES + ADD_BO, H_residual never stored).
// ---------------------------------------------------------------------------
template <typename T, typename TB, int W, int U, bool BI, bool RES, bool ADD_BO, int NT = 0, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void mix_fwd_kernel(const T* __restrict__ H, const TB* __restrict__ bo,
                                                           WRow pre, WRow res, WRow post, T* __restrict__ bi,
                                                           T* __restrict__ out, Geom g) {
  // One workgroup per tile: grid.x == g.ntiles.
  const int64_t b = g.b0 + blockIdx.y;
  const int64_t D = g.D;
  const uint32_t tile = blockIdx.x;
  // Spans start at the tile's first token.
  const int64_t s_lo = (int64_t)(tile * (kThreads * U)) / g.nch;
  const int64_t t0 = b * g.S + s_lo;
  const int64_t rest = g.S - s_lo;
  const Span<T, BUF> hs(H + t0 * 4 * D, rest * 4 * D);
  Frag<T, W> hf[U][4];
  Frag<TB, W> bf[U];
  uint32_t e4[U], e1[U];  // element offsets in the [.,4,D] and [.,D] spans
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile * (kThreads * U) + u * kThreads + threadIdx.x;
    ok[u] = i < g.items;
    const uint32_t s = ok[u] ? i / g.nch : (uint32_t)s_lo;
    const uint32_t c = ok[u] ? i - s * g.nch : 0;
    const uint32_t ds = s - (uint32_t)s_lo;
    e4[u] = ds * 4 * (uint32_t)D + c * W;
    e1[u] = ds * (uint32_t)D + c * W;
    if (ok[u]) {
#pragma unroll
      for (int n = 0; n < 4; ++n) hf[u][n].template load<(NT & 1) != 0>(hs, e4[u] + n * (uint32_t)D);
      if constexpr (ADD_BO) {
        const Span<TB, BUF> bs(bo + t0 * D, rest * D);
        bf[u].template load<(NT & 1) != 0>(bs, e1[u]);
      }
    }
  }
  loads_issued();
  // The weights are fetched behind the tile's loads: waiting for them first
  // cost the closure forward 2.5% (195 -> 190 us at config-3 size).
  float wp[4], wr[16], wq[4];
  if constexpr (BI) load_w4(pre, b, wp);
  if constexpr (RES) load_w16(res, b, wr);
  if constexpr (ADD_BO) load_w4(post, b, wq);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    float h[4][W], bv[W];
#pragma unroll
    for (int n = 0; n < 4; ++n) hf[u][n].unpack(h[n]);
    if constexpr (ADD_BO) bf[u].unpack(bv);
    if constexpr (BI) {
      float r[W];
#pragma unroll
      for (int e = 0; e < W; ++e)
        r[e] = wp[0] * h[0][e] + wp[1] * h[1][e] + wp[2] * h[2][e] + wp[3] * h[3][e];
      const Span<T, BUF> bis(bi + t0 * D, rest * D);
      st<T, W, (NT & 2) != 0>(bis, e1[u], r);
    }
    if constexpr (RES) {
      const Span<T, BUF> os(out + t0 * 4 * D, rest * 4 * D);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        float r[W];
#pragma unroll
        for (int e = 0; e < W; ++e) {
          float v = wr[4 * n] * h[0][e] + wr[4 * n + 1] * h[1][e] + wr[4 * n + 2] * h[2][e] +
                    wr[4 * n + 3] * h[3][e];
          if constexpr (ADD_BO) v += wq[n] * bv[e];
          r[e] = v;
        }
        st<T, W, (NT & 2) != 0>(os, e4[u] + n * (uint32_t)D, r);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Add residual forward from a materialised H_residual (fused_add_residual):
//   out[s,n,:] = hr[s,n,:] + post[n] bo[s,:]
// ---------------------------------------------------------------------------
template <typename T, typename TB, int W, int U, int NT = 0, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void add_residual_fwd_kernel(const T* __restrict__ hr,
                                                                    const TB* __restrict__ bo, WRow post,
                                                                    T* __restrict__ out, Geom g) {
  // One workgroup per tile (grid.x == g.ntiles); the weights are fetched behind the tile's loads.
  const int64_t b = g.b0 + blockIdx.y;
  const int64_t D = g.D;
  const uint32_t tile = blockIdx.x;
  const int64_t s_lo = (int64_t)(tile * (kThreads * U)) / g.nch;
  const int64_t t0 = b * g.S + s_lo;
  const int64_t rest = g.S - s_lo;
  const Span<T, BUF> hs(hr + t0 * 4 * D, rest * 4 * D);
  const Span<TB, BUF> bs(bo + t0 * D, rest * D);
  Frag<T, W> hf[U][4];
  Frag<TB, W> bf[U];
  uint32_t e4[U];
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t i = tile * (kThreads * U) + u * kThreads + threadIdx.x;
    ok[u] = i < g.items;
    const uint32_t s = ok[u] ? i / g.nch : (uint32_t)s_lo;
    const uint32_t c = ok[u] ? i - s * g.nch : 0;
    const uint32_t ds = s - (uint32_t)s_lo;
    e4[u] = ds * 4 * (uint32_t)D + c * W;
    if (ok[u]) {
#pragma unroll
      for (int n = 0; n < 4; ++n) hf[u][n].template load<(NT & 1) != 0>(hs, e4[u] + n * (uint32_t)D);
      bf[u].template load<(NT & 1) != 0>(bs, ds * (uint32_t)D + c * W);
    }
  }
  loads_issued();
  float wq[4];
  load_w4(post, b, wq);
  const Span<T, BUF> os(out + t0 * 4 * D, rest * 4 * D);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    if (!ok[u]) continue;
    float h[4][W], bv[W];
#pragma unroll
    for (int n = 0; n < 4; ++n) hf[u][n].unpack(h[n]);
    bf[u].unpack(bv);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float r[W];
#pragma unroll
      for (int e = 0; e < W; ++e) r[e] = h[n][e] + wq[n] * bv[e];
      st<T, W, (NT & 2) != 0>(os, e4[u] + n * (uint32_t)D, r);
    }
  }
}

// ---------------------------------------------------------------------------
// Add residual backward (fused_add_residual, and the layer closure):
//   d_bo[s,:] = sum_n post[n] dHn[s,n,:]              (written, dtype TB)
//   part[k]   = sum dHn[s,k,:] * bo[s,:]   k < 4      (reduced -> dH_post)
// ---------------------------------------------------------------------------
template <typename T, typename TB, int W, int U, int NT = 0, bool BUF = (W > 1), bool ONE = false>
__global__ __launch_bounds__(kThreads) void add_residual_bwd_kernel(const T* __restrict__ dhn,
                                                                    const TB* __restrict__ bo, WRow post,
                                                                    TB* __restrict__ dbo, float* __restrict__ part,
                                                                    Geom g) {
  // ONE: one workgroup per tile (grid.x == g.ntiles), the weights fetched behind the tile's loads;
  // otherwise workgroups stride over the tiles.
  __shared__ float lds[16 * 4];
  const int64_t b = g.b0 + blockIdx.y;
  float wq[4];
  if constexpr (!ONE) load_w4(post, b, wq);
  const int64_t D = g.D;
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  for (uint32_t tile = blockIdx.x; tile < g.ntiles; tile += gridDim.x) {
    const int64_t s_lo = (int64_t)(tile * (kThreads * U)) / g.nch;
    const int64_t t0 = b * g.S + s_lo;
    const int64_t rest = g.S - s_lo;
    const Span<T, BUF> hs(dhn + t0 * 4 * D, rest * 4 * D);
    const Span<TB, BUF> bs(bo + t0 * D, rest * D);
    const Span<TB, BUF> ds_(dbo + t0 * D, rest * D);
    float h[U][4][W];
    float bv[U][W];
    uint32_t e1[U];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = tile * (kThreads * U) + u * kThreads + threadIdx.x;
      ok[u] = i < g.items;
      const uint32_t s = ok[u] ? i / g.nch : (uint32_t)s_lo;
      const uint32_t c = ok[u] ? i - s * g.nch : 0;
      const uint32_t dt = s - (uint32_t)s_lo;
      e1[u] = dt * (uint32_t)D + c * W;
      if (ok[u]) {
        const uint32_t e4 = dt * 4 * (uint32_t)D + c * W;
#pragma unroll
        for (int n = 0; n < 4; ++n) ld<T, W, (NT & 1) != 0>(hs, e4 + n * (uint32_t)D, h[u][n]);
        ld<TB, W, (NT & 1) != 0>(bs, e1[u], bv[u]);
      }
    }
    if constexpr (ONE) load_w4(post, b, wq);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      float r[W];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        r[e] = wq[0] * h[u][0][e] + wq[1] * h[u][1][e] + wq[2] * h[u][2][e] + wq[3] * h[u][3][e];
#pragma unroll
        for (int n = 0; n < 4; ++n) acc[n] += h[u][n][e] * bv[u][e];
      }
      st<TB, W, (NT & 2) != 0>(ds_, e1[u], r);
    }
    if constexpr (ONE) break;
  }
  const float tot = block_sum_rows<4>(acc, lds);
  if (threadIdx.x < 4) part[(b * gridDim.x + blockIdx.x) * 4 + threadIdx.x] = tot;
}

// ---------------------------------------------------------------------------
// Mixing backward.  With dbi = d branch_input, dhn = d H_residual (or d H_new
// in the layer path, where dH_residual = dH_new):
//   WRITE_DH: dH[s,m,:] = pre[m] dbi + sum_n res[n,m] dhn[s,n,:] (+ gx[m,:] * inv_S)
//   REDUCE:   part[0:4]  = sum dbi * H[s,n,:]          -> dH_pre
//             part[4:20] = sum dhn[s,n,:] * H[s,m,:]   -> dH_res (n-major)
// HAS_DHN = false treats dhn as zero (H_new / H_residual got no gradient).
// (The dynamic layer's dH, which also adds grad_x / S, is dh_kernel.)
// NT bit 2 puts the nt policy on the H loads alone: the dynamic layer's pass B
// reads H for the last time but d_bi and dH_new again in pass C, which then
// finds part of them in the 256 MB memory-side cache.
// ---------------------------------------------------------------------------
template <typename T, int W, int U, bool HAS_DHN, bool REDUCE, bool WRITE_DH, int NT = 0, bool BUF = (W > 1),
          bool ONE = false>
__global__ __launch_bounds__(kThreads) void mix_bwd_kernel(const T* __restrict__ dbi, const T* __restrict__ dhn,
                                                           const T* __restrict__ H, WRow pre, WRow res,
                                                           T* __restrict__ dH, float* __restrict__ part, Geom g) {
  // ONE: one workgroup per tile (grid.x == g.ntiles), the weights fetched behind the tile's loads;
  // otherwise workgroups stride over the tiles.
  __shared__ float lds[16 * 20];
  const int64_t b = g.b0 + blockIdx.y;
  float wp[4], wr[16];
  if constexpr (WRITE_DH && !ONE) {
    load_w4(pre, b, wp);
    if constexpr (HAS_DHN) load_w16(res, b, wr);
  }
  const int64_t D = g.D;
  float acc[20];
#pragma unroll
  for (int k = 0; k < 20; ++k) acc[k] = 0.f;
  for (uint32_t tile = blockIdx.x; tile < g.ntiles; tile += gridDim.x) {
    const int64_t s_lo = (int64_t)(tile * (kThreads * U)) / g.nch;
    const int64_t t0 = b * g.S + s_lo;
    const int64_t rest = g.S - s_lo;
    const Span<T, BUF> dbs(dbi + t0 * D, rest * D);
    const Span<T, BUF> dns(dhn + t0 * 4 * D, rest * 4 * D);
    const Span<T, BUF> hs(H + t0 * 4 * D, rest * 4 * D);
    float db[U][W];
    float dn[U][4][W];
    float h[U][4][W];
    uint32_t e4[U];  // element offset of (s, n=0, c*W) in the [.,4,D] spans
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = tile * (kThreads * U) + u * kThreads + threadIdx.x;
      ok[u] = i < g.items;
      const uint32_t s = ok[u] ? i / g.nch : (uint32_t)s_lo;
      const uint32_t c = ok[u] ? i - s * g.nch : 0;
      const uint32_t dt = s - (uint32_t)s_lo;
      e4[u] = dt * 4 * (uint32_t)D + c * W;
      if (ok[u]) {
        ld<T, W, (NT & 1) != 0>(dbs, dt * (uint32_t)D + c * W, db[u]);
        if constexpr (HAS_DHN) {
#pragma unroll
          for (int n = 0; n < 4; ++n) ld<T, W, (NT & 1) != 0>(dns, e4[u] + n * (uint32_t)D, dn[u][n]);
        }
        if constexpr (REDUCE) {
#pragma unroll
          for (int n = 0; n < 4; ++n) ld<T, W, (NT & 5) != 0>(hs, e4[u] + n * (uint32_t)D, h[u][n]);
        }
      }
    }
    if constexpr (WRITE_DH && ONE) {
      loads_issued();
      load_w4(pre, b, wp);
      if constexpr (HAS_DHN) load_w16(res, b, wr);
    }
    const Span<T, BUF> dHs(dH + t0 * 4 * D, rest * 4 * D);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (!ok[u]) continue;
      if constexpr (REDUCE) {
#pragma unroll
        for (int e = 0; e < W; ++e) {
#pragma unroll
          for (int n = 0; n < 4; ++n) acc[n] += db[u][e] * h[u][n][e];
          if constexpr (HAS_DHN) {
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
              for (int m = 0; m < 4; ++m) acc[4 + 4 * n + m] += dn[u][n][e] * h[u][m][e];
          }
        }
      }
      if constexpr (WRITE_DH) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          float r[W];
#pragma unroll
          for (int e = 0; e < W; ++e) {
            // One fixed fma chain: a zero dH_new term is then an exact no-op,
            // so HAS_DHN with dH_new == 0 gives the same bits as !HAS_DHN.
            float v = wp[m] * db[u][e];
            if constexpr (HAS_DHN) {
#pragma unroll
              for (int n = 0; n < 4; ++n) v = __builtin_fmaf(wr[4 * n + m], dn[u][n][e], v);
            }
            r[e] = v;
          }
          st<T, W, (NT & 2) != 0>(dHs, e4[u] + m * (uint32_t)D, r);
        }
      }
    }
    if constexpr (ONE) break;
  }
  if constexpr (REDUCE) {
    const float tot = block_sum_rows<20>(acc, lds);
    if (threadIdx.x < 20) part[(b * gridDim.x + blockIdx.x) * 20 + threadIdx.x] = tot;
  }
}

// ---------------------------------------------------------------------------
// dH of the dynamic layer (pass C):
//   dH[s,m,:] = pre[m] d_bi[s,:] + sum_n res[n,m] dHn[s,n,:] + grad_x[m,:] / S
// grad_x (f32, [4][D] per batch) is the same for every token, so a lane
// handles one column vector for TT consecutive tokens and loads its grad_x
// slice once: per token it then issues 5 loads instead of 13 (at config-3
// size 212 -> 200 us).  Same arithmetic, in the same order, as the WRITE_DH
// path of mix_bwd_kernel, so the results are bit-identical.
// Items are (token group, column vector) pairs, flattened as in the mixing
// kernels: item i = blockIdx.x * 256 + lane is group i / nch, column i % nch,
// so every lane has work whatever D is (with 256-wide column blocks, D = 7168
// left one block in four half idle: pass C at config 4 ran at 76% of 8 TB/s).
// Grid: x = ceil(groups * nch / 256), y = batch within the launch.
// ---------------------------------------------------------------------------
template <typename T, int W, int TT, bool HAS_DHN, int NT = 0, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void dh_kernel(const T* __restrict__ dbi, const T* __restrict__ dhn,
                                                      const float* __restrict__ gx, float inv_S, WRow pre,
                                                      WRow res, T* __restrict__ dH, int64_t S, int64_t D,
                                                      uint32_t groups, int64_t b0) {
  const int64_t b = b0 + blockIdx.y;
  const uint32_t nch = (uint32_t)(D / W);
  const uint32_t i = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
  const uint32_t grp = i / nch;
  if (grp >= groups) return;
  const int64_t cw = (int64_t)(i - grp * nch) * W;
  // Spans start at the workgroup's first token; dt0 is this lane's token offset in them.
  const int64_t s_lo = (int64_t)((blockIdx.x * (uint32_t)kThreads) / nch) * TT;
  const int64_t s0 = (int64_t)grp * TT;
  const uint32_t dt0 = (uint32_t)(s0 - s_lo);
  const int64_t t0 = b * S + s_lo;
  const int64_t rest = S - s_lo;
  const Span<T, BUF> dbs(dbi + t0 * D, rest * D);
  const Span<T, BUF> dns(dhn + t0 * 4 * D, rest * 4 * D);
  const Span<T, BUF> dHs(dH + t0 * 4 * D, rest * 4 * D);
  float wp[4], wr[16];
  load_w4(pre, b, wp);
  if constexpr (HAS_DHN) load_w16(res, b, wr);
  float gv[4][W];
#pragma unroll
  for (int m = 0; m < 4; ++m) ld<float, W>(gx + b * 4 * D + m * D + cw, gv[m]);
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int64_t s = s0 + t;
    if (s >= S) break;
    const uint32_t dt = dt0 + (uint32_t)t;
    const uint32_t e4 = dt * 4 * (uint32_t)D + (uint32_t)cw;
    Frag<T, W> bf;
    Frag<T, W> nf[4];
    bf.template load<(NT & 1) != 0>(dbs, dt * (uint32_t)D + (uint32_t)cw);
    if constexpr (HAS_DHN) {
#pragma unroll
      for (int n = 0; n < 4; ++n) nf[n].template load<(NT & 1) != 0>(dns, e4 + n * (uint32_t)D);
    }
    loads_issued();
    float db[W], dn[4][W];
    bf.unpack(db);
    if constexpr (HAS_DHN) {
#pragma unroll
      for (int n = 0; n < 4; ++n) nf[n].unpack(dn[n]);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      float r[W];
#pragma unroll
      for (int e = 0; e < W; ++e) {
        float v = wp[m] * db[e];
        if constexpr (HAS_DHN) {
#pragma unroll
          for (int n = 0; n < 4; ++n) v = __builtin_fmaf(wr[4 * n + m], dn[n][e], v);
        }
        r[e] = __builtin_fmaf(gv[m][e], inv_S, v);
      }
      st<T, W, (NT & 2) != 0>(dHs, e4 + m * (uint32_t)D, r);
    }
  }
}

// ---------------------------------------------------------------------------
// The two ends of a hyper-connection stack (no counterpart in the reference,
// whose callers build them from torch ops):
//   expand:   H[s,n,:] = scale * x[s,:]           n = 0..3   (model input)
//   collapse: y[s,:]   = scale * sum_n H[s,n,:]              (model output)
// Each is the other's adjoint with the same scale, so the pair also serves as
// each other's backward.  An item is W consecutive elements of one token row;
// W is the wider 16-byte vector of the two dtypes (or 1 on the ragged path).
// ---------------------------------------------------------------------------
template <typename TX, typename TH, int W, int NT = 0, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void expand_kernel(const TX* __restrict__ x, TH* __restrict__ H,
                                                          float scale, Geom g) {
  const int64_t b = g.b0 + blockIdx.y;
  const int64_t D = g.D;
  for (uint32_t tile = blockIdx.x; tile < g.ntiles; tile += gridDim.x) {
    const int64_t s_lo = (int64_t)(tile * kThreads) / g.nch;
    const int64_t t0 = b * g.S + s_lo;
    const int64_t rest = g.S - s_lo;
    const uint32_t i = tile * kThreads + threadIdx.x;
    if (i >= g.items) continue;
    const uint32_t s = i / g.nch;
    const uint32_t cw = (i - s * g.nch) * W;
    const uint32_t dt = s - (uint32_t)s_lo;
    const Span<TX, BUF> xs(x + t0 * D, rest * D);
    const Span<TH, BUF> hs(H + t0 * 4 * D, rest * 4 * D);
    float v[W];
    ld<TX, W, (NT & 1) != 0>(xs, dt * (uint32_t)D + cw, v);
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] *= scale;
#pragma unroll
    for (int n = 0; n < 4; ++n) st<TH, W, (NT & 2) != 0>(hs, dt * 4 * (uint32_t)D + cw + n * (uint32_t)D, v);
  }
}

template <typename TH, typename TY, int W, int NT = 0, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void collapse_kernel(const TH* __restrict__ H, TY* __restrict__ y,
                                                            float scale, Geom g) {
  const int64_t b = g.b0 + blockIdx.y;
  const int64_t D = g.D;
  for (uint32_t tile = blockIdx.x; tile < g.ntiles; tile += gridDim.x) {
    const int64_t s_lo = (int64_t)(tile * kThreads) / g.nch;
    const int64_t t0 = b * g.S + s_lo;
    const int64_t rest = g.S - s_lo;
    const uint32_t i = tile * kThreads + threadIdx.x;
    const bool ok = i < g.items;
    const uint32_t s = ok ? i / g.nch : (uint32_t)s_lo;
    const uint32_t cw = ok ? (i - s * g.nch) * W : 0;
    const uint32_t dt = s - (uint32_t)s_lo;
    const Span<TH, BUF> hs(H + t0 * 4 * D, rest * 4 * D);
    Frag<TH, W> hf[4];
    if (ok) {
#pragma unroll
      for (int n = 0; n < 4; ++n) hf[n].template load<(NT & 1) != 0>(hs, dt * 4 * (uint32_t)D + cw + n * (uint32_t)D);
    }
    loads_issued();
    if (!ok) continue;
    float h[4][W], r[W];
#pragma unroll
    for (int n = 0; n < 4; ++n) hf[n].unpack(h[n]);
#pragma unroll
    for (int e = 0; e < W; ++e) r[e] = (((h[0][e] + h[1][e]) + h[2][e]) + h[3][e]) * scale;
    const Span<TY, BUF> ys(y + t0 * D, rest * D);
    st<TY, W, (NT & 2) != 0>(ys, dt * (uint32_t)D + cw, r);
  }
}

// Final reduction of [B][nblk][NV] partials into up to two outputs:
// out0[b*SPLIT + k] for k < SPLIT, out1[b*(NV-SPLIT) + k-SPLIT] otherwise.
// Grid: x = batch, y = one 16-byte column (4 consecutive elements) of the
// NV-float records (NV % 4 == 0, 16-byte aligned in the workspace), 1024
// threads per workgroup.  Thread t sums records t, t + 1024, ... in index
// order; each 16-lane row adds its threads' sums with DPP, and threads 0..3
// add the 64 row sums in row order: a fixed order, the same for every column
// split.  (With one batch the closure backward leaves 28672 records at config
// 4; 256 threads took 8.3 us over them.)
constexpr int kRedThreads = 1024;

template <int NV, int SPLIT>
__global__ __launch_bounds__(kRedThreads) void reduce_split_kernel(const float* __restrict__ part,
                                                                   float* __restrict__ out0,
                                                                   float* __restrict__ out1, int nblk) {
  static_assert(NV % 4 == 0, "records of whole 16-byte vectors");
  constexpr int kRows = kRedThreads / 16;
  __shared__ float lds[kRows * 4];
  const int64_t b = blockIdx.x;
  const int q = blockIdx.y;
  const f32x4* p = reinterpret_cast<const f32x4*>(part + b * nblk * NV) + q;
  f32x4 a4 = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int k = threadIdx.x; k < nblk; k += kRedThreads) a4 += p[(int64_t)k * (NV / 4)];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const float v = sum_all16(a4[c]);
    if ((threadIdx.x & 15) == 0) lds[(threadIdx.x >> 4) * 4 + c] = v;
  }
  __syncthreads();
  if (threadIdx.x < 4) {
    const int c = threadIdx.x;
    float t = 0.f;
#pragma unroll 8
    for (int r = 0; r < kRows; ++r) t += lds[r * 4 + c];
    const int i = 4 * q + c;
    if (i < SPLIT) out0[b * SPLIT + i] = t;
    else out1[b * (NV - SPLIT) + (i - SPLIT)] = t;
  }
}

// reduce_split_kernel for at most 16 partials per batch (many short sequences: at S = 1,
// D = 4096 the closure backward leaves two per batch, and 4096 batches of 1024-thread
// workgroups took 11.3 us): one 16-lane row per (batch, 16-byte column).  The same sums in the
// same order -- the row's DPP tree, added to zero, as in reduce_split_kernel, whose other rows
// then hold zeros -- so the same bits.  Every lane of a row runs the DPP sums.
template <int NV, int SPLIT>
__global__ __launch_bounds__(kThreads) void reduce_split_small_kernel(const float* __restrict__ part,
                                                                      float* __restrict__ out0,
                                                                      float* __restrict__ out1, int nblk,
                                                                      int64_t B) {
  constexpr int NQ = NV / 4;
  const int64_t g = ((int64_t)blockIdx.x * kThreads + threadIdx.x) >> 4;  // (batch, column) pair
  const int k = threadIdx.x & 15;
  const bool ok = g < B * NQ;
  const int64_t b = ok ? g / NQ : 0;
  const int q = ok ? (int)(g - b * NQ) : 0;
  f32x4 a4 = f32x4{0.f, 0.f, 0.f, 0.f};
  if (ok && k < nblk) a4 += reinterpret_cast<const f32x4*>(part + b * nblk * NV)[(int64_t)k * NQ + q];
  float v[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) v[c] = sum_all16(a4[c]);
  if (ok && k < 4) {
    const float t = 0.f + (k == 0 ? v[0] : k == 1 ? v[1] : k == 2 ? v[2] : v[3]);
    const int i = 4 * q + k;
    if (i < SPLIT) out0[b * SPLIT + i] = t;
    else out1[b * (NV - SPLIT) + (i - SPLIT)] = t;
  }
}

// ---------------------------------------------------------------------------
// Host-side launch helpers.
// ---------------------------------------------------------------------------

// The final reduce of nblk partial records of NV floats per batch (see reduce_split_kernel).
template <int NV, int SPLIT>
inline hipError_t launch_reduce_split(const float* part, float* out0, float* out1, int nblk, int64_t B,
                                      hipStream_t st) {
  if (nblk <= 16) {
    const unsigned nwg = (unsigned)((B * (NV / 4) * 16 + kThreads - 1) / kThreads);
    reduce_split_small_kernel<NV, SPLIT><<<dim3(nwg), kThreads, 0, st>>>(part, out0, out1, nblk, B);
  } else {
    reduce_split_kernel<NV, SPLIT><<<dim3((unsigned)B, NV / 4), kRedThreads, 0, st>>>(part, out0, out1, nblk);
  }
  return hipGetLastError();
}

// True when every pointer is 16-byte aligned and D splits into whole 16-byte
// vectors of every dtype involved.  The vector path addresses through
// per-workgroup buffer spans (Span): a tile of up to 2 * 256 items touches at
// most 2 + 4096 / nch tokens (dh_kernel: 2), i.e. under (16384 + 8 D) elements
// of a [., 4, D] tensor, which must stay below 2^31 bytes for fp32.
inline bool vec_ok(int64_t D, int W, std::initializer_list<const void*> ptrs) {
  if (D % W != 0) return false;
  if (!span_ok(16384 + 8 * D, 4)) return false;
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

// Workgroups per batch for a reduction kernel: about kRedBlocks in total
// (8 per CU on a 256-CU MI355X), never more than there are tiles.  The cap is
// a constant so workspace sizes do not depend on the device.
constexpr int64_t kRedBlocks = 2048;

inline uint32_t reduce_blocks(uint32_t ntiles, int64_t B) {
  int64_t per_b = kRedBlocks / (B > 0 ? B : 1);
  if (per_b > (int64_t)ntiles) per_b = ntiles;
  if (per_b < 1) per_b = 1;
  return (uint32_t)per_b;
}

// Bytes of partial sums a reduction kernel over B batches may write.
inline size_t partial_bytes(int64_t B, int nv) {
  const int64_t per_b = kRedBlocks / (B > 0 ? B : 1) > 1 ? kRedBlocks / (B > 0 ? B : 1) : 1;
  return (size_t)(B * per_b * nv) * sizeof(float);
}

// Bytes of the partials of a reduction kernel that runs one workgroup per tile
// on the vector path (nv floats per workgroup) and the reduce_blocks count on
// the ragged path.  Sized for the narrowest vector width (fp32, 4 elements per
// lane, one item per lane), because the path is chosen per call from the
// pointers' alignment.
inline size_t tile_partial_bytes(int64_t B, int64_t S, int64_t D, int nv) {
  const int64_t tiles = (S * D / 4 + kThreads - 1) / kThreads;
  const size_t vec = (size_t)(B > 0 ? B : 1) * (size_t)(tiles > 0 ? tiles : 1) * nv * sizeof(float);
  const size_t rag = partial_bytes(B, nv);
  return vec > rag ? vec : rag;
}

// Launch fn(b0, nb) for consecutive batch chunks that fit grid.y.
template <class F>
inline int for_batch_chunks(int64_t B, F&& fn) {
  for (int64_t b0 = 0; b0 < B; b0 += kMaxGridY) {
    const int64_t nb = (B - b0) < kMaxGridY ? (B - b0) : kMaxGridY;
    if (int rc = fn(b0, nb)) return rc;
  }
  return MHC_OK;
}

// Checks the common (B, S, D) constraints of the streaming kernels.
inline int check_bsd(const char* who, int64_t B, int64_t S, int64_t D) {
  if (B < 0 || S < 0 || D < 0) {
    set_error("%s: negative size (B=%lld S=%lld D=%lld)", who, (long long)B, (long long)S, (long long)D);
    return MHC_ERR_ARG;
  }
  // Per-batch element indices are 32-bit, and a tile's first index (a multiple
  // of 256 items of up to 2 elements each) must stay below 2^32 as well.
  if (S * D > ((int64_t)1 << 32) - ((int64_t)1 << 16)) {
    set_error("%s: S*D = %lld exceeds the per-batch limit of 2^32 - 2^16 elements", who, (long long)(S * D));
    return MHC_ERR_ARG;
  }
  return MHC_OK;
}

}  // namespace mhc

// Nested dispatch over two bulk dtypes: T for the stream tensor, TB for
// branch_output.
#define MHC_DISPATCH_DTYPE2(dtype_a, dtype_b, ...)                      \
  MHC_DISPATCH_DTYPE(dtype_a, [&] {                                     \
    using TA_ = T;                                                      \
    return MHC_DISPATCH_DTYPE(dtype_b, [&] {                            \
      using TB = T;                                                     \
      using TH = TA_;                                                   \
      return __VA_ARGS__();                                             \
    });                                                                 \
  })
