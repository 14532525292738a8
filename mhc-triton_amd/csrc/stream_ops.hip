// Entry points of the low-level stream ops: fused_stream_mix and
// fused_add_residual, forward and backward (reference src/mhc/_kernels.py:617-687,
// src/mhc/_backward.py:533-626).
#include "stream_kernels.hpp"

namespace mhc {

constexpr int kU = 1;  // items per lane per tile

template <typename T, int W>
static int stream_mix_fwd(const T* H, const float* pre, const float* res, T* bi, T* out, int64_t B, int64_t S,
                          int64_t D, hipStream_t st) {
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, kU>(S, D, b0);
    if (g.ntiles == 0) return (int)MHC_OK;
    mix_fwd_kernel<T, T, W, kU, true, true, false, kNt><<<dim3(g.ntiles, nb), kThreads, occupancy_lds(2), st>>>(
        H, (const T*)nullptr, WRow{pre, 4}, WRow{res, 16}, WRow{nullptr, 0}, bi, out, g);
    return hip_status(hipGetLastError(), "stream_mix_forward launch");
  });
}

template <typename T, int W>
static int stream_mix_bwd(const T* dbi, const T* dhr, const T* H, const float* pre, const float* res, T* dH,
                          float* dpre, float* dres, int64_t B, int64_t S, int64_t D, float* part,
                          hipStream_t st) {
  // Vector path: one workgroup per tile, weights fetched behind its loads, up
  // to 6 per CU, a partial per tile.  Ragged path: workgroups stride over the
  // tiles at 3 per CU.
  const Geom g0 = make_geom<W, kU>(S, D, 0);
  const uint32_t nblk = W > 1 ? g0.ntiles : reduce_blocks(g0.ntiles, B);
  // With no tiles nothing is launched and the reduce writes zeros.
  int rc = nblk == 0 ? (int)MHC_OK : for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, kU>(S, D, b0);
    if constexpr (W > 1)
      mix_bwd_kernel<T, W, kU, true, true, true, kNt, true, true><<<dim3(nblk, nb), kThreads, occupancy_lds(6), st>>>(
          dbi, dhr, H, WRow{pre, 4}, WRow{res, 16}, dH, part, g);
    else
      mix_bwd_kernel<T, W, kU, true, true, true, kNt><<<dim3(nblk, nb), kThreads, occupancy_lds(3), st>>>(
          dbi, dhr, H, WRow{pre, 4}, WRow{res, 16}, dH, part, g);
    return hip_status(hipGetLastError(), "stream_mix_backward launch");
  });
  if (rc) return rc;
  return hip_status(launch_reduce_split<20, 4>(part, dpre, dres, (int)nblk, B, st),
                    "stream_mix_backward reduce launch");
}

template <typename TH, typename TB, int W>
static int add_res_fwd(const TH* hr, const TB* bo, const float* post, TH* out, int64_t B, int64_t S, int64_t D,
                       hipStream_t st) {
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, kU>(S, D, b0);
    if (g.ntiles == 0) return (int)MHC_OK;
    add_residual_fwd_kernel<TH, TB, W, kU, kNt><<<dim3(g.ntiles, nb), kThreads, occupancy_lds(4), st>>>(
        hr, bo, WRow{post, 4}, out, g);
    return hip_status(hipGetLastError(), "add_residual_forward launch");
  });
}

template <typename TH, typename TB, int W>
static int add_res_bwd(const TH* dhn, const TB* bo, WRow post, TB* dbo, float* dpost, int64_t B, int64_t S,
                       int64_t D, float* part, hipStream_t st) {
  // Vector path: one workgroup per tile at 4 per CU (the closure backward at
  // config-3 size: 134 -> 128 us against 512 looping workgroups per batch at
  // 2 per CU).  Ragged path: a capped count of looping workgroups.
  const Geom g0 = make_geom<W, kU>(S, D, 0);
  // At least one workgroup: with no tiles it writes zero partials, so dH_post comes out zero.
  uint32_t nblk = W > 1 ? g0.ntiles : reduce_blocks(g0.ntiles, B);
  if (nblk == 0) nblk = 1;
  int rc = for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, kU>(S, D, b0);
    if constexpr (W > 1)
      add_residual_bwd_kernel<TH, TB, W, kU, kNt, true, true><<<dim3(nblk, nb), kThreads, occupancy_lds(4), st>>>(
          dhn, bo, post, dbo, part, g);
    else
      add_residual_bwd_kernel<TH, TB, W, kU, kNt><<<dim3(nblk, nb), kThreads, occupancy_lds(2), st>>>(
          dhn, bo, post, dbo, part, g);
    return hip_status(hipGetLastError(), "add_residual_backward launch");
  });
  if (rc) return rc;
  return hip_status(launch_reduce_split<4, 4>(part, dpost, nullptr, (int)nblk, B, st),
                    "add_residual_backward reduce launch");
}

template <typename TH, typename TB>
static constexpr int wide_w() {
  return Vec<TH>::N > Vec<TB>::N ? Vec<TH>::N : Vec<TB>::N;
}

int check_workspace(const char* who, const void* ws, size_t have, size_t need) {
  if (need == 0) return MHC_OK;
  if (!ws || have < need) {
    set_error("%s: workspace of %zu bytes required, %zu given", who, need, ws ? have : (size_t)0);
    return MHC_ERR_WORKSPACE;
  }
  if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) {
    set_error("%s: workspace must be 256-byte aligned", who);
    return MHC_ERR_WORKSPACE;
  }
  return MHC_OK;
}

// Exposed to the layer entry points (layer.hip).
template <typename TH, typename TB>
int add_residual_backward_t(const void* dhn, const void* bo, WRow post, void* dbo, float* dpost, int64_t B,
                            int64_t S, int64_t D, float* part, hipStream_t st) {
  constexpr int WV = wide_w<TH, TB>();
  if (vec_ok(D, WV, {dhn, bo, dbo}))
    return add_res_bwd<TH, TB, WV>((const TH*)dhn, (const TB*)bo, post, (TB*)dbo, dpost, B, S, D, part, st);
  return add_res_bwd<TH, TB, 1>((const TH*)dhn, (const TB*)bo, post, (TB*)dbo, dpost, B, S, D, part, st);
}

int add_residual_backward_any(const void* dhn, int dtype_h, const void* bo, int dtype_bo, WRow post, void* dbo,
                              float* dpost, int64_t B, int64_t S, int64_t D, float* part, hipStream_t st) {
  return MHC_DISPATCH_DTYPE2(dtype_h, dtype_bo, [&] {
    return add_residual_backward_t<TH, TB>(dhn, bo, post, dbo, dpost, B, S, D, part, st);
  });
}

}  // namespace mhc

using namespace mhc;

extern "C" int mhc_stream_mix_forward(const void* H, const float* H_pre, const float* H_res, void* branch_input,
                                      void* H_residual, int64_t B, int64_t S, int64_t D, int dtype,
                                      mhc_stream_t stream) {
  if (int rc = check_bsd("stream_mix_forward", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!H || !H_pre || !H_res || !branch_input || !H_residual) {
    set_error("stream_mix_forward: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    constexpr int WV = Vec<T>::N;
    if (vec_ok(D, WV, {H, branch_input, H_residual}))
      return stream_mix_fwd<T, WV>((const T*)H, H_pre, H_res, (T*)branch_input, (T*)H_residual, B, S, D, st);
    return stream_mix_fwd<T, 1>((const T*)H, H_pre, H_res, (T*)branch_input, (T*)H_residual, B, S, D, st);
  });
}

extern "C" size_t mhc_stream_mix_backward_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype) {
  (void)S; (void)D; (void)dtype;
  return tile_partial_bytes(B, S, D, 20);
}

extern "C" int mhc_stream_mix_backward(const void* d_branch_input, const void* dH_residual, const void* H,
                                       const float* H_pre, const float* H_res, void* dH, float* dH_pre,
                                       float* dH_res, int64_t B, int64_t S, int64_t D, int dtype, void* workspace,
                                       size_t workspace_bytes, mhc_stream_t stream) {
  if (int rc = check_bsd("stream_mix_backward", B, S, D)) return rc;
  if (B == 0) return MHC_OK;
  if (S * D == 0) {  // empty sums: zero weight gradients, dH is empty
    if (!dH_pre || !dH_res) {
      set_error("stream_mix_backward: null pointer");
      return MHC_ERR_ARG;
    }
    if (int rc = fill_zero(dH_pre, B * 4, (hipStream_t)stream)) return rc;
    return fill_zero(dH_res, B * 16, (hipStream_t)stream);
  }
  if (!d_branch_input || !dH_residual || !H || !H_pre || !H_res || !dH || !dH_pre || !dH_res) {
    set_error("stream_mix_backward: null pointer");
    return MHC_ERR_ARG;
  }
  if (int rc = check_workspace("stream_mix_backward", workspace, workspace_bytes,
                               mhc_stream_mix_backward_workspace_bytes(B, S, D, dtype)))
    return rc;
  hipStream_t st = (hipStream_t)stream;
  float* part = (float*)workspace;
  return MHC_DISPATCH_DTYPE(dtype, [&] {
    constexpr int WV = Vec<T>::N;
    if (vec_ok(D, WV, {d_branch_input, dH_residual, H, dH}))
      return stream_mix_bwd<T, WV>((const T*)d_branch_input, (const T*)dH_residual, (const T*)H, H_pre, H_res,
                                   (T*)dH, dH_pre, dH_res, B, S, D, part, st);
    return stream_mix_bwd<T, 1>((const T*)d_branch_input, (const T*)dH_residual, (const T*)H, H_pre, H_res,
                                (T*)dH, dH_pre, dH_res, B, S, D, part, st);
  });
}

extern "C" int mhc_add_residual_forward(const void* H_residual, int dtype_h, const void* branch_output,
                                        int dtype_bo, const float* H_post, void* H_new, int64_t B, int64_t S,
                                        int64_t D, mhc_stream_t stream) {
  if (int rc = check_bsd("add_residual_forward", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!H_residual || !branch_output || !H_post || !H_new) {
    set_error("add_residual_forward: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  return MHC_DISPATCH_DTYPE2(dtype_h, dtype_bo, [&] {
    constexpr int WV = wide_w<TH, TB>();
    if (vec_ok(D, WV, {H_residual, branch_output, H_new}))
      return add_res_fwd<TH, TB, WV>((const TH*)H_residual, (const TB*)branch_output, H_post, (TH*)H_new, B, S, D,
                                     st);
    return add_res_fwd<TH, TB, 1>((const TH*)H_residual, (const TB*)branch_output, H_post, (TH*)H_new, B, S, D,
                                  st);
  });
}

extern "C" size_t mhc_add_residual_backward_workspace_bytes(int64_t B, int64_t S, int64_t D, int dtype_h) {
  (void)dtype_h;
  return tile_partial_bytes(B, S, D, 4);
}

extern "C" int mhc_add_residual_backward(const void* dH_new, int dtype_h, const void* branch_output, int dtype_bo,
                                         const float* H_post, void* d_branch_output, float* dH_post, int64_t B,
                                         int64_t S, int64_t D, void* workspace, size_t workspace_bytes,
                                         mhc_stream_t stream) {
  if (int rc = check_bsd("add_residual_backward", B, S, D)) return rc;
  if (B == 0) return MHC_OK;
  if (S * D == 0) {  // empty sums: zero dH_post, d_branch_output is empty
    if (!dH_post) {
      set_error("add_residual_backward: null pointer");
      return MHC_ERR_ARG;
    }
    return fill_zero(dH_post, B * 4, (hipStream_t)stream);
  }
  if (!dH_new || !branch_output || !H_post || !d_branch_output || !dH_post) {
    set_error("add_residual_backward: null pointer");
    return MHC_ERR_ARG;
  }
  if (int rc = check_workspace("add_residual_backward", workspace, workspace_bytes,
                               mhc_add_residual_backward_workspace_bytes(B, S, D, dtype_h)))
    return rc;
  return add_residual_backward_any(dH_new, dtype_h, branch_output, dtype_bo, WRow{H_post, 4}, d_branch_output,
                                   dH_post, B, S, D, (float*)workspace, (hipStream_t)stream);
}

namespace mhc {

template <typename TX, typename TH, int W>
static int expand_launch(const TX* x, TH* H, float scale, int64_t B, int64_t S, int64_t D, hipStream_t st) {
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, 1>(S, D, b0);
    // nt stores only: with nt on its one load this write-dominated kernel runs 10% slower.
    expand_kernel<TX, TH, W, 2><<<dim3(g.ntiles, nb), kThreads, occupancy_lds(2), st>>>(x, H, scale, g);
    return hip_status(hipGetLastError(), "stream_expand launch");
  });
}

template <typename TH, typename TY, int W>
static int collapse_launch(const TH* H, TY* y, float scale, int64_t B, int64_t S, int64_t D, hipStream_t st) {
  return for_batch_chunks(B, [&](int64_t b0, int64_t nb) {
    const Geom g = make_geom<W, 1>(S, D, b0);
    collapse_kernel<TH, TY, W, kNt><<<dim3(g.ntiles, nb), kThreads, occupancy_lds(4), st>>>(H, y, scale, g);
    return hip_status(hipGetLastError(), "stream_collapse launch");
  });
}

}  // namespace mhc

extern "C" int mhc_stream_expand(const void* x, int dtype_x, void* H, int dtype_h, int64_t B, int64_t S, int64_t D,
                                 float scale, mhc_stream_t stream) {
  if (int rc = check_bsd("stream_expand", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!x || !H) {
    set_error("stream_expand: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  // TH: the stream tensor's dtype, TB: x's dtype.
  return MHC_DISPATCH_DTYPE2(dtype_h, dtype_x, [&] {
    constexpr int WV = wide_w<TH, TB>();
    if (vec_ok(D, WV, {x, H})) return expand_launch<TB, TH, WV>((const TB*)x, (TH*)H, scale, B, S, D, st);
    return expand_launch<TB, TH, 1>((const TB*)x, (TH*)H, scale, B, S, D, st);
  });
}

extern "C" int mhc_stream_collapse(const void* H, int dtype_h, void* y, int dtype_y, int64_t B, int64_t S,
                                   int64_t D, float scale, mhc_stream_t stream) {
  if (int rc = check_bsd("stream_collapse", B, S, D)) return rc;
  if (B * S * D == 0) return MHC_OK;
  if (!H || !y) {
    set_error("stream_collapse: null pointer");
    return MHC_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  // TH: the stream tensor's dtype, TB: y's dtype.
  return MHC_DISPATCH_DTYPE2(dtype_h, dtype_y, [&] {
    constexpr int WV = wide_w<TH, TB>();
    if (vec_ok(D, WV, {H, y})) return collapse_launch<TH, TB, WV>((const TH*)H, (TB*)y, scale, B, S, D, st);
    return collapse_launch<TH, TB, 1>((const TH*)H, (TB*)y, scale, B, S, D, st);
  });
}
