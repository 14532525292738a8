// HyperConnection layer path (reference src/mhc/module.py:103-182 composed with
// ops.py / _kernels.py / _backward.py).
//
// Forward, dynamic:   meanpool<PROJ> (reads H)  -> finalize (weights w[B,24])
//                     -> branch_input pass (reads H, writes bi)
// Closure forward:    H_new = H_res @ H + H_post * bo (reads H, bo; writes H_new)
// Closure backward:   d_bo, dH_post (reads dH_new, bo; writes d_bo)
// Backward, dynamic:  pass B reductions dH_pre, dH_res (reads d_bi, dH_new, H)
//                     -> weights backward (rows, wide: grad_x, grad_phi; sums)
//                     -> pass C: dH = H_pre d_bi + H_res^T dH_new + grad_x / S
//                        (reads d_bi, dH_new; writes dH)
// Per token that is 18 D e bytes forward and 24 D e backward (e = element
// size), against 22 + ~39 for the reference's op-by-op composition.
// Static layers skip the mean-pool and fold pass B into pass C.
#include <mutex>

#include "dynw_kernels.hpp"
#include "stream_kernels.hpp"

namespace mhc {

int check_workspace(const char* who, const void* ws, size_t have, size_t need);
int add_residual_backward_any(const void* dhn, int dtype_h, const void* bo, int dtype_bo, WRow post, void* dbo,
                              float* dpost, int64_t B, int64_t S, int64_t D, float* part, hipStream_t st);
int mean_pool_any(const void* H, int dtype, float* x, const float* phi, float* projpart, float* colpart,
                  int64_t B, int64_t S, int64_t D, int* nrc, hipStream_t st);
size_t mean_pool_colpart_bytes(int dtype, int64_t B, int64_t S, int64_t D);
bool dynw_project_rows_ok(int64_t R, int64_t K, const void* x, int dtype);
int dynw_project_rows(const void* x, int dtype, const float* phi, float* part, int64_t R, int64_t K, int* nK,
                      hipStream_t st);
size_t dynw_grad_split_bytes(int64_t R, int64_t K);
int dynw_grad_pass(const void* x, int dtype_x, const float* phi, const float* rowbuf, void* grad_x, bool gx_f32,
                   float* grad_phi, float* grad_bias, float* grad_alpha, int64_t R, int64_t K, char* split_ws,
                   hipStream_t st);

// Batches from which the dynamic weights of the layer run as the op runs them for rows in bulk.
// Below them the batch is a handful of rows: the projection folds into the mean-pool's reduce
// (which re-reads phi for every batch) and the backward runs one row chunk on the VALU, whose
// latency is what counts there.  At B = 4096, S = 1, D = 4096 the folded projection took 397 us
// and the one-chunk backward 1842 us.  Measured crossovers (graph-replayed steps at D = 4096):
// the backward on the MFMA kernel in row chunks wins from 64 batches on (fwd+bwd 69 -> 59 us at
// B = 64, 2504 -> 622 us at B = 4096).  The projection on the MFMA kernel: at S = 1, where it
// reads H's rows and no mean-pool runs, from 64 batches (no-grad forward with the closure / training
// step: B = 96 27.1 -> 24.2 / 61.1 -> 58.5 us, B = 256 42.2 -> 27.3 / 91.0 -> 73.7; equal at 64);
// for S > 1, after a mean-pool without it, from 64 batches once B * D reaches 2^19: the folded
// projection re-reads phi (4 D x 24 floats) for every batch, so the crossover scales with B * D
// (B = 256, S = 8: 88.1 -> 79.9 / 190.4 -> 183.5; B = 128, S = 16: 82.1 -> 76.5 / 181.1 ->
// 175.8; B = 80, S = 32, D = 7168: 141.0 -> 135.9 / 317.6 -> 310.8; at B = 128, S = 4 the
// forward lost 1.7 us and the step gained 1.6; below 2^19, at B = 128, D = 2048, S = 4 it lost:
// 26.8 -> 29.6 / 67.6 -> 69.8).
constexpr int64_t kLayerBulkRows = 64;
constexpr int64_t kLayerBulkProjRowsS1 = 64;
constexpr int64_t kLayerBulkProjElems = (int64_t)1 << 19;  // B * D

constexpr int kLU = 1;   // items per lane per tile, streaming passes
constexpr int kLRU = 2;  // items per lane per tile, the reduction-only pass B

static size_t al(size_t v) { return (v + 255) & ~(size_t)255; }

// Workspace layout shared by all layer entry points (each uses a prefix of it).
struct LayerWs {
  size_t colpart;    // mean-pool column partials [B][nS][4D]
  size_t pool_part;  // projection partials [B][nrc][25]
  size_t red_part;   // [B][nblk][20] (pass B), [B][tiles][20] (pass BC) or [B][tiles][4] (closure backward)
  size_t dpre;       // [B][4]
  size_t dres;       // [B][16]
  size_t rowbuf;     // [B][52]
  size_t gx;         // [B][4D] grad of the pooled rows (backward); a forward without x at many
                     // batches and S > 1 keeps its pooled rows here
  size_t grad_split; // B >= kLayerBulkRows: the weights backward's row-chunk partials
  size_t total;
};

static LayerWs layer_ws(int64_t B, int64_t S, int64_t D, int dtype) {
  LayerWs w;
  const int64_t nrc = (4 * D + kThreads - 1) / kThreads;
  size_t o = 0;
  w.colpart = o;   o += al(mean_pool_colpart_bytes(dtype, B, S, D));
  w.pool_part = o; o += al((size_t)B * (nrc > 0 ? nrc : 1) * kPart * sizeof(float));
  {
    // the partials of pass B, pass BC and the closure backward share the region
    w.red_part = o;  o += al(tile_partial_bytes(B, S, D, 20));
  }
  w.dpre = o;      o += al((size_t)B * 4 * sizeof(float));
  w.dres = o;      o += al((size_t)B * 16 * sizeof(float));
  w.rowbuf = o;    o += al((size_t)B * kRow * sizeof(float));
  w.gx = o;        o += al((size_t)B * 4 * D * sizeof(float));
  w.grad_split = o; o += B >= kLayerBulkRows ? al(dynw_grad_split_bytes(B, 4 * D)) : 0;
  w.total = o;
  return w;
}

template <typename T, int W>
static int launch_bi(const T* H, const float* w, T* bi, int64_t B, int64_t S, int64_t D, hipStream_t st) {
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, kLU>(S, D, b0);
    if (g.ntiles == 0) return (int)MHC_OK;
    mix_fwd_kernel<T, T, W, kLU, true, false, false, kNt><<<dim3(g.ntiles, nb), kThreads, occupancy_lds(3), st>>>(
        H, (const T*)nullptr, WRow{w, kOut}, WRow{nullptr, 0}, WRow{nullptr, 0}, bi, nullptr, g);
    return hip_status(hipGetLastError(), "layer branch_input launch");
  });
}

static int branch_input_any(const void* H, int dtype, const float* w, void* bi, int64_t B, int64_t S, int64_t D,
                            hipStream_t st) {
  if (S * D == 0) return MHC_OK;
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    constexpr int WV = Vec<T>::N;
    if (vec_ok(D, WV, {H, bi})) return launch_bi<T, WV>((const T*)H, w, (T*)bi, B, S, D, st);
    return launch_bi<T, 1>((const T*)H, w, (T*)bi, B, S, D, st);
  });
}

// Static weights (module.py:108-117), replicated for every batch row:
// H_post = sigmoid(b_post), H_pre = sigmoid(b_pre)/(sum + 1e-8),
// H_res = Sinkhorn(H_res_base, iters, eps = 1e-8).  The 24 values are the same
// for every row: lanes 0..15 of wave 0 form them (16-lane Sinkhorn) in LDS,
// then the workgroup writes its rows.
__global__ __launch_bounds__(kThreads) void static_weights_kernel(const float* __restrict__ bpre,
                                                                  const float* __restrict__ bpost,
                                                                  const float* __restrict__ bres,
                                                                  float* __restrict__ w, int64_t B, int iters) {
  __shared__ float vals[kOut];
  if (threadIdx.x < 16) {
    const int e = threadIdx.x;
    const int j = e & 3;
    vals[8 + e] = sk16_forward(bres[e], iters, 1e-8f);
    const bool is_pre = (e & 4) == 0;
    const float sg = sigmoidf(is_pre ? bpre[j] : bpost[j]);
    const float den = sum_row16(sg) + 1e-8f;  // quad 0: the four H_pre sigmoids
    if (e < 4) vals[j] = sg / den;
    else if (e < 8) vals[4 + j] = sg;
  }
  __syncthreads();
  const int64_t b0 = (int64_t)blockIdx.x * kThreads;
  for (int i = threadIdx.x; i < kThreads * kOut; i += kThreads) {
    const int64_t b = b0 + i / kOut;
    if (b < B) w[b0 * kOut + i] = vals[i % kOut];
  }
}

// Backward of static_weights_kernel through the batch expand:
// every cotangent is first summed over b (fixed order), then pushed through
// sigmoid / normalise / Sinkhorn once (the Sinkhorn VJP is linear in the
// cotangent), on lanes 0..15 in 16-lane form.
__global__ __launch_bounds__(kThreads) void static_weights_bwd_kernel(
    const float* __restrict__ bpre, const float* __restrict__ bpost, const float* __restrict__ bres,
    const float* __restrict__ w, const float* __restrict__ dpre, const float* __restrict__ dpost,
    const float* __restrict__ dres, float* __restrict__ gbias, int64_t B, int iters) {
  __shared__ float lds[4 * kOut];
  __shared__ float tot[kOut];
  __shared__ float slots[kSkSlots * 16];
  float acc[kOut];
#pragma unroll
  for (int j = 0; j < kOut; ++j) acc[j] = 0.f;
  for (int64_t b = threadIdx.x; b < B; b += kThreads) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] += dpre[b * 4 + j];
    if (dpost) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[4 + j] += dpost[b * 4 + j];
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[8 + j] += dres[b * 16 + j];
  }
  block_sum<kOut>(acc, lds);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 0; j < kOut; ++j) tot[j] = acc[j];
  }
  __syncthreads();
  if (threadIdx.x >= 16) return;
  const int e = threadIdx.x;
  const int j = e & 3;
  gbias[8 + e] = iters == 20 ? sk16_backward_fixed<20>(bres[e], tot[8 + e], 1e-8f)
                             : sk16_backward<kSkSlots>(bres[e], tot[8 + e], iters, 1e-8f, slots + e, 16);
  const bool is_pre = (e & 4) == 0;
  const float sg = sigmoidf(is_pre ? bpre[j] : bpost[j]);
  const float den = sum_row16(sg) + 1e-8f;
  const float dot = sum_row16(tot[j] * w[j]);  // quad 0: <g_pre, H_pre>
  if (e < 4) gbias[j] = (tot[j] - dot) / den * sg * (1.f - sg);
  else if (e < 8) gbias[4 + j] = tot[4 + j] * sg * (1.f - sg);
}

// Pass B (REDUCE only), the static pass BC (REDUCE + WRITE_DH) and the
// generic mix backward share mix_bwd_kernel.
template <typename T, int W, bool HAS_DHN, bool REDUCE, bool WRITE_DH>
static int launch_mix_bwd(const T* dbi, const T* dhn, const T* H, const float* w, T* dH, float* part, int64_t B,
                          int64_t S, int64_t D, uint32_t* nblk_out, hipStream_t st) {
  // Pass B writes nothing bulk: two items per lane, full occupancy, workgroups
  // striding over the tiles.  The passes that write dH take one item per lane;
  // on the vector path one workgroup per tile with the weights fetched behind
  // its loads, up to 6 per CU (static pass BC at config-3 size 285.7 -> 280.2
  // us, at config-5 size 298.7 -> 263.6 us), and a partial per tile.
  constexpr int U = WRITE_DH ? kLU : kLRU;
  constexpr bool ONE = WRITE_DH && W > 1;
  const size_t lds = WRITE_DH ? occupancy_lds(ONE ? 6 : (REDUCE ? 3 : 4)) : 0;
  const Geom g0 = make_geom<W, U>(S, D, 0);
  const uint32_t nblk = REDUCE && !ONE ? reduce_blocks(g0.ntiles, B) : g0.ntiles;
  if (nblk_out) *nblk_out = nblk;
  if (nblk == 0) return MHC_OK;
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, U>(S, D, b0);
    // Pass B (REDUCE only): nt on the H loads alone; d_bi and dH_new are read again by pass C.
    constexpr int NT = WRITE_DH ? kNt : 4;
    mix_bwd_kernel<T, W, U, HAS_DHN, REDUCE, WRITE_DH, NT, (W > 1), ONE><<<dim3(nblk, nb), kThreads, lds, st>>>(
        dbi, dhn, H, WRow{w, kOut}, WRow{w + 8, kOut}, dH, part, g);
    return hip_status(hipGetLastError(), "layer mix backward launch");
  });
}

template <typename T, bool REDUCE, bool WRITE_DH>
static int mix_bwd_dispatch(const void* dbi, const void* dhn, const void* H, const float* w, void* dH, float* part,
                            int64_t B, int64_t S, int64_t D, uint32_t* nblk, hipStream_t st) {
  constexpr int WV = Vec<T>::N;
  const bool vec = vec_ok(D, WV, {dbi, dhn, H, dH});
  if (dhn) {
    if (vec)
      return launch_mix_bwd<T, WV, true, REDUCE, WRITE_DH>((const T*)dbi, (const T*)dhn, (const T*)H, w, (T*)dH,
                                                           part, B, S, D, nblk, st);
    return launch_mix_bwd<T, 1, true, REDUCE, WRITE_DH>((const T*)dbi, (const T*)dhn, (const T*)H, w, (T*)dH, part,
                                                        B, S, D, nblk, st);
  }
  if (vec)
    return launch_mix_bwd<T, WV, false, REDUCE, WRITE_DH>((const T*)dbi, nullptr, (const T*)H, w, (T*)dH, part, B,
                                                          S, D, nblk, st);
  return launch_mix_bwd<T, 1, false, REDUCE, WRITE_DH>((const T*)dbi, nullptr, (const T*)H, w, (T*)dH, part, B, S,
                                                       D, nblk, st);
}

// Pass C of the dynamic backward: TT tokens per lane, grad_x loaded once for all of them, 2
// workgroups per CU.  Two tokens measured best at config-3 size (eight: 5 us slower per step).
// A short sequence fits in one group instead, or two at S <= 16, so that grad_x is read once or
// twice per batch rather than S / 2 times (training steps, D = 4096 bf16, two tokens -> dh_tokens:
// S = 3 292.8 -> 283.6 us, S = 4 331.7 -> 323.9, S = 5 327.6 -> 317.5, S = 8 307.5 -> 295.1,
// S = 16 313.9 -> 307.8; at S = 32 and 64 eight tokens gained 1-2 us).  The same arithmetic per
// element: the same bits for every choice.  Only while the grid keeps at least 1024 workgroups
// (four per CU): at B = 64, S = 8 eight tokens left 128 and the step took 80.8 us against 79.5;
// at 256 workgroups the larger groups went either way (B = 128, S = 8: 2.7 us less; B = 64,
// S = 16: 1.7 us more).
static int dh_tokens(int64_t B, int64_t S, int64_t D, int W) {
  for (int tt = S <= 2 ? 2 : (S <= 4 ? 4 : (S <= 16 ? 8 : 2)); tt > 2; tt /= 2)
    if (B * ((S + tt - 1) / tt) * (D / W) >= 1024 * (int64_t)kThreads) return tt;
  return 2;
}

template <typename T, int W, bool HAS_DHN, int TT>
static int launch_dh(const T* dbi, const T* dhn, const float* gx, const float* w, T* dH, int64_t B, int64_t S,
                     int64_t D, hipStream_t st) {
  const int64_t groups = (S + TT - 1) / TT;
  const int64_t items = groups * (D / W);  // (token group, column vector) pairs, < 2^32 by check_bsd
  if (items == 0) return MHC_OK;
  const unsigned nwg = (unsigned)((items + kThreads - 1) / kThreads);
  const float inv_S = 1.f / (float)S;
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    dh_kernel<T, W, TT, HAS_DHN, kNt><<<dim3(nwg, (unsigned)nb), kThreads, occupancy_lds(2), st>>>(
        dbi, dhn, gx, inv_S, WRow{w, kOut}, WRow{w + 8, kOut}, dH, S, D, (uint32_t)groups, b0);
    return hip_status(hipGetLastError(), "layer dH launch");
  });
}

template <typename T, int W, bool HAS_DHN>
static int launch_dh_tt(int tt, const T* dbi, const T* dhn, const float* gx, const float* w, T* dH, int64_t B,
                        int64_t S, int64_t D, hipStream_t st) {
  if (tt == 8) return launch_dh<T, W, HAS_DHN, 8>(dbi, dhn, gx, w, dH, B, S, D, st);
  if (tt == 4) return launch_dh<T, W, HAS_DHN, 4>(dbi, dhn, gx, w, dH, B, S, D, st);
  return launch_dh<T, W, HAS_DHN, 2>(dbi, dhn, gx, w, dH, B, S, D, st);
}

template <typename T>
static int dh_dispatch(const void* dbi, const void* dhn, const float* gx, const float* w, void* dH, int64_t B,
                       int64_t S, int64_t D, hipStream_t st) {
  constexpr int WV = Vec<T>::N;
  const bool vec = vec_ok(D, WV, {dbi, dhn, dH}) && aligned16(gx);
  int tt = dh_tokens(B, S, D, vec ? WV : 1);
  // a tile's buffer spans grow with the tokens per lane (vec_ok bounds them for two)
  if (vec && !span_ok(tt / 2 * (16384 + 8 * D), 4)) tt = 2;
  if (dhn) {
    if (vec) return launch_dh_tt<T, WV, true>(tt, (const T*)dbi, (const T*)dhn, gx, w, (T*)dH, B, S, D, st);
    return launch_dh_tt<T, 1, true>(tt, (const T*)dbi, (const T*)dhn, gx, w, (T*)dH, B, S, D, st);
  }
  if (vec) return launch_dh_tt<T, WV, false>(tt, (const T*)dbi, nullptr, gx, w, (T*)dH, B, S, D, st);
  return launch_dh_tt<T, 1, false>(tt, (const T*)dbi, nullptr, gx, w, (T*)dH, B, S, D, st);
}

}  // namespace mhc

using namespace mhc;

extern "C" size_t mhc_layer_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype) {
  if (B <= 0) return 0;
  return layer_ws(B, S, D, dtype).total;
}

#define LAYER_WS_CHECK(who)                                                                 \
  const LayerWs L = layer_ws(B, S, D, dtype);                                               \
  if (int rc_ = check_workspace(who, workspace, workspace_bytes, L.total)) return rc_;      \
  char* wsb = (char*)workspace;

// Argument checks shared by the two dynamic-forward entry points; 0 when the call may proceed
// (also for B == 0, which the callers then return early on).
static int layer_dynamic_forward_args(const char* who, const void* H, const float* phi, const float* H_pre_base,
                                      const float* H_post_base, const float* H_res_base, const float* alpha_pre,
                                      const float* alpha_post, const float* alpha_res, const void* branch_input,
                                      const float* x, const float* w, const float* aux, int64_t B, int64_t S,
                                      int64_t D, int iters) {
  if (int rc = check_bsd(who, B, S, D)) return rc;
  if (iters < 0) { set_error("%s: negative iters", who); return MHC_ERR_ARG; }
  if (B == 0) return MHC_OK;
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!H || !branch_input)) || !phi || !H_pre_base || !H_post_base || !H_res_base || !alpha_pre ||
      !alpha_post || !alpha_res || !w || !aux) {
    set_error("%s: null pointer", who);
    return MHC_ERR_ARG;
  }
  return MHC_OK;
}

// The dynamic layer forward proper: mean-pool with the projection partials, the Eq. 14-19
// epilogue, branch_input.  It uses the column partials (L.colpart) and the projection
// partials (L.pool_part) of the workspace at wsb, and overwrites every entry it reads.
static int layer_dynamic_forward_run(const void* H, int dtype, const float* phi, const float* H_pre_base,
                                     const float* H_post_base, const float* H_res_base, const float* alpha_pre,
                                     const float* alpha_post, const float* alpha_res, void* branch_input, float* x,
                                     float* w, float* aux, int64_t B, int64_t S, int64_t D, int iters, float eps,
                                     const LayerWs& L, char* wsb, bool full_ws, hipStream_t st) {
  float* part = (float*)(wsb + L.pool_part);
  int nK = 0;
  const int64_t K = 4 * D;
  DynParams P{H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res};
  // Many batches: the mean-pool alone, then the pooled rows' projection on MFMA (its records
  // fit the projection-partial region: at most K / 512 chunks against K / 256).  At S = 1 the
  // pooled rows are H's own rows, projected as they are (half the bytes of the f32 rows in
  // 16-bit H), and the f32 copy is written only for a backward that asks for it.  For S > 1
  // without x (no backward follows) the pooled rows go to the workspace's grad_x region, so
  // that the weights come out as with x; only a caller without the full workspace (the
  // allocation-free entry) then takes the folded projection below.
  const bool s1 = S == 1 && dynw_project_rows_ok(B, K, H, dtype);
  float* xp = x ? x : (full_ws ? (float*)(wsb + L.gx) : nullptr);
  if (s1 ? B >= kLayerBulkProjRowsS1
         : (B >= kLayerBulkRows && B * D >= kLayerBulkProjElems && xp &&
            dynw_project_rows_ok(B, K, xp, MHC_DTYPE_F32))) {
    if (x || !s1)
      if (int rc = mean_pool_any(H, dtype, xp, nullptr, nullptr, (float*)(wsb + L.colpart), B, S, D, nullptr, st))
        return rc;
    if (int rc = s1 ? dynw_project_rows(H, dtype, phi, part, B, K, &nK, st)
                    : dynw_project_rows(xp, MHC_DTYPE_F32, phi, part, B, K, &nK, st))
      return rc;
    dynw_finalize_rows_kernel<><<<dim3((unsigned)((B + kFinRowsWg - 1) / kFinRowsWg)), kThreads, 0, st>>>(
        part, nK, B, K, P, OutRow{w, kOut}, OutRow{w + 4, kOut}, OutRow{w + 8, kOut}, aux, iters, eps);
    if (int rc = hip_status(hipGetLastError(), "layer finalize launch")) return rc;
    return branch_input_any(H, dtype, w, branch_input, B, S, D, st);
  }
  if (int rc = mean_pool_any(H, dtype, x, phi, part, (float*)(wsb + L.colpart), B, S, D, &nK, st)) return rc;
  dynw_finalize_kernel<><<<dim3((unsigned)((B + 3) / 4)), kThreads, 0, st>>>(
      part, nK, B, K, P, OutRow{w, kOut}, OutRow{w + 4, kOut}, OutRow{w + 8, kOut}, aux, iters, eps);
  if (int rc = hip_status(hipGetLastError(), "layer finalize launch")) return rc;
  return branch_input_any(H, dtype, w, branch_input, B, S, D, st);
}

extern "C" int mhc_layer_dynamic_forward(const void* H, int dtype, const float* phi, const float* H_pre_base,
                                         const float* H_post_base, const float* H_res_base,
                                         const float* alpha_pre, const float* alpha_post, const float* alpha_res,
                                         void* branch_input, float* x, float* w, float* aux, int64_t B, int64_t S,
                                         int64_t D, int iters, float eps, void* workspace, size_t workspace_bytes,
                                         mhc_stream_t stream) {
  if (int rc = layer_dynamic_forward_args("layer_dynamic_forward", H, phi, H_pre_base, H_post_base, H_res_base,
                                          alpha_pre, alpha_post, alpha_res, branch_input, x, w, aux, B, S, D,
                                          iters))
    return rc;
  if (B == 0) return MHC_OK;
  LAYER_WS_CHECK("layer_dynamic_forward");
  return layer_dynamic_forward_run(H, dtype, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post,
                                   alpha_res, branch_input, x, w, aux, B, S, D, iters, eps, L, wsb, true,
                                   (hipStream_t)stream);
}

// ---------------------------------------------------------------------------
// Allocation-free dynamic layer forward.  Its scratch is the static device
// array below: every GPU the library runs on holds its own copy, for the life
// of the process.  In host code `scratch` only names the symbol; the device
// address of each GPU's copy comes from hipGetSymbolAddress, taken once per
// device with that device current, and kept in g_scratch_dev.  Calls that
// overlap on one GPU (different streams) share the array and race.  The kept
// address is never refreshed: hipDeviceReset on a GPU where the entry point
// has run invalidates it, and the header rules out calls after one.
// ---------------------------------------------------------------------------
constexpr size_t kScratchBytes = MHC_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_dev[kMaxDevices];

// Device address of the current device's scratch array.
static int scratch_on_current_device(char** out) {
  int dev = -1;
  if (int rc = hip_status(hipGetDevice(&dev), "layer_dynamic_forward_noalloc: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) {
    set_error("layer_dynamic_forward_noalloc: device %d beyond the %d the library tracks", dev, kMaxDevices);
    return MHC_ERR_ARG;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    if (int rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                            "layer_dynamic_forward_noalloc: hipGetSymbolAddress"))
      return rc;
    if (!p || ((uintptr_t)p & 255) != 0) {
      set_error("layer_dynamic_forward_noalloc: scratch address %p is not 256-byte aligned", p);
      return MHC_ERR_HIP;
    }
    g_scratch_dev[dev] = p;
  }
  *out = (char*)g_scratch_dev[dev];
  return MHC_OK;
}

extern "C" int mhc_layer_dynamic_forward_noalloc(const void* H, int dtype, const float* phi,
                                                 const float* H_pre_base, const float* H_post_base,
                                                 const float* H_res_base, const float* alpha_pre,
                                                 const float* alpha_post, const float* alpha_res,
                                                 void* branch_input, float* x, float* w, float* aux, int64_t B,
                                                 int64_t S, int64_t D, int iters, float eps, mhc_stream_t stream) {
  const char* who = "layer_dynamic_forward_noalloc";
  if (int rc = layer_dynamic_forward_args(who, H, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post,
                                          alpha_res, branch_input, x, w, aux, B, S, D, iters))
    return rc;
  if (B == 0) return MHC_OK;
  // The forward reads and writes only the column and projection partials, which
  // lead the layer workspace: its first L.red_part bytes.
  const LayerWs L = layer_ws(B, S, D, dtype);
  if (L.red_part > kScratchBytes) {
    set_error("%s: B=%lld S=%lld D=%lld needs %zu bytes of scratch, more than the %zu the static array holds; "
              "call mhc_layer_dynamic_forward with a workspace instead",
              who, (long long)B, (long long)S, (long long)D, L.red_part, kScratchBytes);
    return MHC_ERR_WORKSPACE;
  }
  char* wsb = nullptr;
  if (int rc = scratch_on_current_device(&wsb)) return rc;
  return layer_dynamic_forward_run(H, dtype, phi, H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post,
                                   alpha_res, branch_input, x, w, aux, B, S, D, iters, eps, L, wsb, false,
                                   (hipStream_t)stream);
}

extern "C" int mhc_layer_static_forward(const void* H, int dtype, const float* H_pre_base, const float* H_post_base,
                                        const float* H_res_base, void* branch_input, float* w, int64_t B,
                                        int64_t S, int64_t D, int iters, mhc_stream_t stream) {
  if (int rc = check_bsd("layer_static_forward", B, S, D)) return rc;
  if (iters < 0) { set_error("layer_static_forward: negative iters"); return MHC_ERR_ARG; }
  if (B == 0) return MHC_OK;
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!H || !branch_input)) || !H_pre_base || !H_post_base || !H_res_base || !w) {
    set_error("layer_static_forward: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  static_weights_kernel<<<dim3((unsigned)((B + kThreads - 1) / kThreads)), kThreads, 0, st>>>(
      H_pre_base, H_post_base, H_res_base, w, B, iters);
  if (int rc = hip_status(hipGetLastError(), "static weights launch")) return rc;
  return branch_input_any(H, dtype, w, branch_input, B, S, D, st);
}

extern "C" int mhc_layer_add_forward(const void* H, int dtype_h, const void* branch_output, int dtype_bo,
                                     const float* w, void* H_new, int64_t B, int64_t S, int64_t D,
                                     mhc_stream_t stream) {
  if (int rc = check_bsd("layer_add_forward", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!H || !branch_output || !w || !H_new) {
    set_error("layer_add_forward: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  return MHC_DISPATCH_DTYPE2(dtype_h, dtype_bo, [&] {
    constexpr int WV = Vec<TH>::N > Vec<TB>::N ? Vec<TH>::N : Vec<TB>::N;
    auto go = [&](auto wtag) {
      constexpr int W = decltype(wtag)::value;
      return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
        const Geom g = make_geom<W, kLU>(S, D, b0);
        // 3 workgroups per CU: 188.5 us at config-3 size against 194.9 with 2 and 190.4 with 4
        // when chosen; with the buffer-span loads and nt policy caps 2 and 3 time alike and 4
        // is about 1 us slower (192.6-195.4 us event-timed in the bench).
        mix_fwd_kernel<TH, TB, W, kLU, false, true, true, kNt>
            <<<dim3(g.ntiles, nb), kThreads, occupancy_lds(3), st>>>(
            (const TH*)H, (const TB*)branch_output, WRow{nullptr, 0}, WRow{w + 8, kOut}, WRow{w + 4, kOut},
            nullptr, (TH*)H_new, g);
        return hip_status(hipGetLastError(), "layer add forward launch");
      });
    };
    if (vec_ok(D, WV, {H, branch_output, H_new})) return go(std::integral_constant<int, WV>{});
    return go(std::integral_constant<int, 1>{});
  });
}

extern "C" int mhc_layer_add_backward(const void* dH_new, int dtype_h, const void* branch_output, int dtype_bo,
                                      const float* w, void* d_branch_output, float* dH_post, int64_t B, int64_t S,
                                      int64_t D, void* workspace, size_t workspace_bytes, mhc_stream_t stream) {
  const int dtype = dtype_h;
  if (int rc = check_bsd("layer_add_backward", B, S, D)) return rc;
  if (B == 0) return MHC_OK;
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!dH_new || !branch_output || !d_branch_output)) || !w || !dH_post) {
    set_error("layer_add_backward: null pointer");
    return MHC_ERR_ARG;
  }
  LAYER_WS_CHECK("layer_add_backward");
  return add_residual_backward_any(dH_new, dtype_h, branch_output, dtype_bo, WRow{w + 4, kOut}, d_branch_output,
                                   dH_post, B, S, D, (float*)(wsb + L.red_part), (hipStream_t)stream);
}

extern "C" int mhc_layer_dynamic_backward(const void* H, int dtype, const void* d_branch_input, const void* dH_new,
                                          const float* dH_post, const float* phi, const float* H_pre_base,
                                          const float* H_post_base, const float* H_res_base,
                                          const float* alpha_pre, const float* alpha_post,
                                          const float* alpha_res, const float* x, const float* w,
                                          const float* aux, void* dH, float* grad_phi, float* grad_bias,
                                          float* grad_alpha, int64_t B, int64_t S, int64_t D, int iters, float eps,
                                          void* workspace, size_t workspace_bytes, mhc_stream_t stream) {
  if (int rc = check_bsd("layer_dynamic_backward", B, S, D)) return rc;
  if (iters < 0) { set_error("layer_dynamic_backward: negative iters"); return MHC_ERR_ARG; }
  if (B == 0) {
    // No rows: every parameter gradient is an empty sum.
    hipStream_t st = (hipStream_t)stream;
    if (grad_phi)
      if (int rc = fill_zero(grad_phi, 4 * D * kOut, st)) return rc;
    if (grad_bias)
      if (int rc = fill_zero(grad_bias, kOut, st)) return rc;
    return grad_alpha ? fill_zero(grad_alpha, 3, st) : MHC_OK;
  }
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!H || !d_branch_input)) || !phi || !H_pre_base || !H_post_base || !H_res_base || !alpha_pre ||
      !alpha_post || !alpha_res || (!x && S != 1) || !w || !aux) {
    set_error("layer_dynamic_backward: null pointer");
    return MHC_ERR_ARG;
  }
  LAYER_WS_CHECK("layer_dynamic_backward");
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)(wsb + L.red_part);
  float* rowbuf = (float*)(wsb + L.rowbuf);
  float* gx = (float*)(wsb + L.gx);
  // Pass B: dH_pre, dH_res.
  uint32_t nblk = 0;
  int rc = MHC_DISPATCH_DTYPE(dtype, [&] {
    return mix_bwd_dispatch<T, true, false>(d_branch_input, dH_new, H, w, nullptr, part, B, S, D,
                                                   &nblk, st);
  });
  if (rc) return rc;
  // Weights backward: the rows kernel sums the pass-B partials itself; the wide
  // kernel also sums grad_bias / grad_alpha.
  DynParams P{H_pre_base, H_post_base, H_res_base, alpha_pre, alpha_post, alpha_res};
  const int64_t K = 4 * D;
  // A workgroup per batch sums up to thousands of partials (B = 1: 2048); with at most 64 per
  // batch (from 32 batches on) one wave's lanes hold them all, so a workgroup takes four batches,
  // a wave each, and adds the same four 16-lane row sums in the same order (B = 4096, S = 1:
  // 16.0 us for one batch per workgroup, whose Sinkhorn backward then keeps 16 of 64 lanes busy).
  if (nblk <= 64)
    dynw_bwd_rows_kernel<4><<<dim3((unsigned)((B + 3) / 4)), kThreads, 0, st>>>(
        aux, P, InRow{w, kOut}, InRow{nullptr, 0}, InRow{dH_post, 4}, InRow{nullptr, 0}, part, (int)nblk, rowbuf,
        B, K, iters, eps);
  else
    dynw_bwd_rows_kernel<1><<<dim3((unsigned)B), kThreads, 0, st>>>(
        aux, P, InRow{w, kOut}, InRow{nullptr, 0}, InRow{dH_post, 4}, InRow{nullptr, 0}, part, (int)nblk, rowbuf,
        B, K, iters, eps);
  if ((rc = hip_status(hipGetLastError(), "layer weights backward rows launch"))) return rc;
  // The pooled rows: x, or without it (S = 1) H's own rows, read in H's dtype; grad_x stays f32.
  const void* xr = x ? (const void*)x : H;
  const int xdt = x ? MHC_DTYPE_F32 : dtype;
  if (B >= kLayerBulkRows)
    rc = dynw_grad_pass(xr, xdt, phi, rowbuf, dH ? gx : nullptr, true, grad_phi, grad_bias, grad_alpha, B, K,
                        wsb + L.grad_split, st);
  else
    rc = MHC_DISPATCH_DTYPE(xdt, [&] {
      return hip_status(launch_dynw_bwd_wide<T, float>((const T*)xr, phi, rowbuf, dH ? gx : nullptr, grad_phi,
                                                       nullptr, grad_bias, grad_alpha, B, K, B, 1u, aligned16(phi),
                                                       st),
                        "layer weights backward wide launch");
    });
  if (rc) return rc;
  if (!dH || S * D == 0) return MHC_OK;
  // Pass C: dH.
  return MHC_DISPATCH_DTYPE(dtype, [&] { return dh_dispatch<T>(d_branch_input, dH_new, gx, w, dH, B, S, D, st); });
}

extern "C" int mhc_layer_static_backward(const void* H, int dtype, const void* d_branch_input, const void* dH_new,
                                         const float* dH_post, const float* H_pre_base, const float* H_post_base,
                                         const float* H_res_base, const float* w, void* dH, float* grad_bias,
                                         int64_t B, int64_t S, int64_t D, int iters, void* workspace,
                                         size_t workspace_bytes, mhc_stream_t stream) {
  if (int rc = check_bsd("layer_static_backward", B, S, D)) return rc;
  if (iters < 0) { set_error("layer_static_backward: negative iters"); return MHC_ERR_ARG; }
  if (B == 0) return grad_bias ? fill_zero(grad_bias, kOut, (hipStream_t)stream) : MHC_OK;  // empty sums
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!H || !d_branch_input)) || !H_pre_base || !H_post_base || !H_res_base || !w || !grad_bias) {
    set_error("layer_static_backward: null pointer");
    return MHC_ERR_ARG;
  }
  LAYER_WS_CHECK("layer_static_backward");
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)(wsb + L.red_part);
  float* dpre = (float*)(wsb + L.dpre);
  float* dres = (float*)(wsb + L.dres);
  // Pass BC: reductions and dH in one sweep.
  uint32_t nblk = 0;
  int rc = MHC_DISPATCH_DTYPE(dtype, [&] {
    if (dH)
      return mix_bwd_dispatch<T, true, true>(d_branch_input, dH_new, H, w, dH, part, B, S, D, &nblk,
                                                    st);
    return mix_bwd_dispatch<T, true, false>(d_branch_input, dH_new, H, w, nullptr, part, B, S, D,
                                                   &nblk, st);
  });
  if (rc) return rc;
  rc = hip_status(launch_reduce_split<20, 4>(part, dpre, dres, (int)nblk, B, st), "layer static reduce launch");
  if (rc) return rc;
  static_weights_bwd_kernel<<<1, kThreads, 0, st>>>(H_pre_base, H_post_base, H_res_base, w, dpre, dH_post, dres,
                                                    grad_bias, B, iters);
  return hip_status(hipGetLastError(), "static weights backward launch");
}

extern "C" int mhc_layer_branch_input(const void* H, int dtype, const float* w, void* branch_input, int64_t B,
                                      int64_t S, int64_t D, mhc_stream_t stream) {
  if (int rc = check_bsd("layer_branch_input", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!H || !w || !branch_input) {
    set_error("layer_branch_input: null pointer");
    return MHC_ERR_ARG;
  }
  return branch_input_any(H, dtype, w, branch_input, B, S, D, (hipStream_t)stream);
}

extern "C" int mhc_layer_mix_backward(const void* H, int dtype, const void* d_branch_input, const void* dH_new,
                                      const float* w, void* dH, float* dH_pre, float* dH_res, int64_t B,
                                      int64_t S, int64_t D, void* workspace, size_t workspace_bytes,
                                      mhc_stream_t stream) {
  if (int rc = check_bsd("layer_mix_backward", B, S, D)) return rc;
  if (B == 0) return MHC_OK;
  const bool nz = S * D != 0;  // bulk tensors may be empty (null) when S * D == 0
  if ((nz && (!H || !d_branch_input)) || !w || !dH_pre || !dH_res) {
    set_error("layer_mix_backward: null pointer");
    return MHC_ERR_ARG;
  }
  LAYER_WS_CHECK("layer_mix_backward");
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)(wsb + L.red_part);
  uint32_t nblk = 0;
  int rc = MHC_DISPATCH_DTYPE(dtype, [&] {
    if (dH)
      return mix_bwd_dispatch<T, true, true>(d_branch_input, dH_new, H, w, dH, part, B, S, D, &nblk,
                                                    st);
    return mix_bwd_dispatch<T, true, false>(d_branch_input, dH_new, H, w, nullptr, part, B, S, D,
                                                   &nblk, st);
  });
  if (rc) return rc;
  return hip_status(launch_reduce_split<20, 4>(part, dH_pre, dH_res, (int)nblk, B, st),
                    "layer mix backward reduce launch");
}

extern "C" int mhc_layer_mix_dh(const void* d_branch_input, const void* dH_new, int dtype, const float* w,
                                const float* grad_x, void* dH, int64_t B, int64_t S, int64_t D,
                                mhc_stream_t stream) {
  if (int rc = check_bsd("layer_mix_dh", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!d_branch_input || !w || !grad_x || !dH) {
    set_error("layer_mix_dh: null pointer");
    return MHC_ERR_ARG;
  }
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    return dh_dispatch<T>(d_branch_input, dH_new, grad_x, w, dH, B, S, D, (hipStream_t)stream);
  });
}
