// Shared device helpers for the gfx950 mHC kernels.
//
// Bulk tensors (H, branch_input, H_residual, branch_output and their
// gradients) are stored as fp32, bf16 or fp16 and always computed in fp32.
// Every streaming kernel moves 16 bytes per lane per access
// (global_load_dwordx4 / global_store_dwordx4): 4 fp32 or 8 bf16/fp16
// elements.  Small per-batch weights (H_pre, H_post, H_res: 24 floats) are
// fp32 and are read through the scalar cache because the batch index is
// uniform across a workgroup (blockIdx.y).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/mhc_abi.h"

namespace mhc {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

constexpr int kThreads = 256;  // 4 waves of 64 lanes

// Elements per 16-byte access.
template <typename T> struct Vec { static constexpr int N = 16 / sizeof(T); };

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16 <- f32 and f16 <- f32 round to nearest even, the
// same rounding torch uses for .to(bfloat16) / .to(float16); gfx950 has
// v_cvt_pk_bf16_f32 for the former.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(__bf16 v) { return (float)v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return (float)v; }

template <typename T> __device__ __forceinline__ T from_f32(float v);
template <> __device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <> __device__ __forceinline__ __bf16 from_f32<__bf16>(float v) { return (__bf16)v; }
template <> __device__ __forceinline__ _Float16 from_f32<_Float16>(float v) { return (_Float16)v; }

// ---------------------------------------------------------------------------
// 16-byte vector load / store with conversion to / from fp32.
// ---------------------------------------------------------------------------
template <typename T> struct Io;

// `NT` loads and stores carry the non-temporal hint (streamed data that this
// kernel touches once): on gfx950 they are issued with the streaming cache
// policy, which measurably raises HBM throughput of pure streaming kernels.
template <typename V>
__device__ __forceinline__ V vload(const V* p, bool nt) {
  return nt ? __builtin_nontemporal_load(p) : *p;
}

template <> struct Io<float> {
  template <bool NT = false>
  __device__ __forceinline__ static void load(const float* p, float* f) {
    f32x4 v = vload(reinterpret_cast<const f32x4*>(p), NT);
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
  template <bool NT>
  __device__ __forceinline__ static void store(float* p, const float* f) {
    f32x4 v = {f[0], f[1], f[2], f[3]};
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
    else *reinterpret_cast<f32x4*>(p) = v;
  }
};

template <> struct Io<__bf16> {
  template <bool NT = false>
  __device__ __forceinline__ static void load(const __bf16* p, float* f) {
    u32x4 r = vload(reinterpret_cast<const u32x4*>(p), NT);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(r[i] << 16);
      f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
  template <bool NT>
  __device__ __forceinline__ static void store(__bf16* p, const float* f) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 pair = {f[2 * i], f[2 * i + 1]};
      r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pair, bf16x2));
    }
    if constexpr (NT) __builtin_nontemporal_store(r, reinterpret_cast<u32x4*>(p));
    else *reinterpret_cast<u32x4*>(p) = r;
  }
};

template <> struct Io<_Float16> {
  template <bool NT = false>
  __device__ __forceinline__ static void load(const _Float16* p, float* f) {
    const f16x8 v = vload(reinterpret_cast<const f16x8*>(p), NT);
    const f32x8 w = __builtin_convertvector(v, f32x8);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = w[i];
  }
  template <bool NT>
  __device__ __forceinline__ static void store(_Float16* p, const float* f) {
    f32x8 w;
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = f[i];
    const f16x8 v = __builtin_convertvector(w, f16x8);
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f16x8*>(p));
    else *reinterpret_cast<f16x8*>(p) = v;
  }
};

// Raw 16-byte vector of each bulk type, its unpacking to fp32 and the
// packing of 16 bytes' worth of fp32 values (rounded as from_f32 does).
template <typename T> struct RawVec;
template <> struct RawVec<float> {
  using type = f32x4;
  __device__ __forceinline__ static void unpack(const type& v, float* f) {
    f[0] = v.x; f[1] = v.y; f[2] = v.z; f[3] = v.w;
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    return __builtin_bit_cast(u32x4, (f32x4{f[0], f[1], f[2], f[3]}));
  }
};
template <> struct RawVec<__bf16> {
  using type = u32x4;
  __device__ __forceinline__ static void unpack(const type& r, float* f) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = __uint_as_float(r[i] << 16);
      f[2 * i + 1] = __uint_as_float(r[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f32x2 pair = {f[2 * i], f[2 * i + 1]};
      r[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector(pair, bf16x2));
    }
    return r;
  }
};
template <> struct RawVec<_Float16> {
  using type = f16x8;
  __device__ __forceinline__ static void unpack(const type& v, float* f) {
    const f32x8 w = __builtin_convertvector(v, f32x8);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = w[i];
  }
  __device__ __forceinline__ static u32x4 pack(const float* f) {
    f32x8 w;
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = f[i];
    return __builtin_bit_cast(u32x4, __builtin_convertvector(w, f16x8));
  }
};

// ---------------------------------------------------------------------------
// Addressing of a streamed tensor from one workgroup.  On the 16-byte vector
// path (BUF) loads and stores go through a buffer resource: the span's base
// address in SGPRs, 32-bit per-lane byte offsets, a range check against the
// span's size (loads past it return 0, stores past it are dropped), and the
// streaming (nt) cache policy where the caller asks for it.  Against 64-bit
// global addresses this drops the per-access address arithmetic and lets the
// nt policy apply to loads too: the closure forward runs at 81% of 8 TB/s
// instead of 77%.  The W = 1 (ragged) path keeps a plain pointer.  Offsets
// are in elements from the span's base; the host keeps a workgroup's span
// under 2^31 bytes (span_ok).  The resource's third dword (raw, 32-bit data
// format) is the gfx9-family value.
// ---------------------------------------------------------------------------
constexpr int kBufRsrcDword3 = 0x00020000;

template <typename T, bool BUF>
struct Span;

template <typename T>
struct Span<T, true> {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ Span(const T* base, int64_t elems) {
    int64_t bytes = elems * (int64_t)sizeof(T);
    bytes = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
    r = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(base), 0, (int)bytes, kBufRsrcDword3);
  }
  template <bool NT>
  __device__ __forceinline__ u32x4 load16(uint32_t e) const {
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)(e * (uint32_t)sizeof(T)), 0, NT ? 2 : 0);
  }
  template <bool NT>
  __device__ __forceinline__ uint32_t load4(uint32_t e) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)(e * (uint32_t)sizeof(T)), 0, NT ? 2 : 0);
  }
  template <bool NT>
  __device__ __forceinline__ void store16(uint32_t e, u32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)(e * (uint32_t)sizeof(T)), 0, NT ? 2 : 0);
  }
};

template <typename T>
struct Span<T, false> {
  T* p;
  __device__ __forceinline__ Span(const T* base, int64_t) : p(const_cast<T*>(base)) {}
};

// A workgroup's span of one tensor must stay under 2^31 bytes on the buffer
// path; `span_elems` is the largest span (in elements) a launch can give it.
inline bool span_ok(int64_t span_elems, int64_t elem_size) {
  return span_elems >= 0 && span_elems * elem_size < ((int64_t)1 << 31);
}

// W consecutive elements of T held as raw 16-byte vectors until unpacked
// (W a multiple of the vector width), or as fp32 on the scalar W = 1 path.
// Kernels issue every load of a tile into fragments first and unpack after:
// with load and unpack interleaved per row the compiler starts unpacking
// early rows before the last loads are issued, and fewer bytes are in flight
// (the closure forward ran 5% slower).
template <typename T, int W>
struct Frag {
  static constexpr int N = Vec<T>::N;
  static constexpr bool kVec = W >= N;
  using Raw = typename RawVec<T>::type;
  Raw r[kVec ? W / N : 1];
  float s[kVec ? 1 : W];

  template <bool NT = false>
  __device__ __forceinline__ void load(const T* p) {
    if constexpr (kVec) {
#pragma unroll
      for (int q = 0; q < W / N; ++q) r[q] = vload(reinterpret_cast<const Raw*>(p + q * N), NT);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) s[i] = to_f32(p[i]);
    }
  }

  template <bool NT, bool BUF>
  __device__ __forceinline__ void load(const Span<T, BUF>& sp, uint32_t e) {
    if constexpr (BUF) {
      static_assert(kVec, "the buffer path moves 16-byte vectors");
#pragma unroll
      for (int q = 0; q < W / N; ++q) r[q] = __builtin_bit_cast(Raw, sp.template load16<NT>(e + q * N));
    } else {
      load<NT>(sp.p + e);
    }
  }

  __device__ __forceinline__ void unpack(float* f) const {
    if constexpr (kVec) {
#pragma unroll
      for (int q = 0; q < W / N; ++q) RawVec<T>::unpack(r[q], f + q * N);
    } else {
#pragma unroll
      for (int i = 0; i < W; ++i) f[i] = s[i];
    }
  }
};

// Load W consecutive elements when W is a multiple of the 16-byte vector
// width of T (several 16-byte loads), or W == 1.
template <typename T, int W, bool NT = false>
__device__ __forceinline__ void ld(const T* p, float* f) {
  constexpr int N = Vec<T>::N;
  if constexpr (W >= N) {
#pragma unroll
    for (int q = 0; q < W / N; ++q) Io<T>::template load<NT>(p + q * N, f + q * N);
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) f[i] = to_f32(p[i]);
  }
}

template <typename T, int W, bool NT = false>
__device__ __forceinline__ void st(T* p, const float* f) {
  constexpr int N = Vec<T>::N;
  if constexpr (W >= N) {
#pragma unroll
    for (int q = 0; q < W / N; ++q) Io<T>::template store<NT>(p + q * N, f + q * N);
  } else {
#pragma unroll
    for (int i = 0; i < W; ++i) p[i] = from_f32<T>(f[i]);
  }
}

// The same through a Span (element offset e from the span's base).
template <typename T, int W, bool NT, bool BUF>
__device__ __forceinline__ void st(const Span<T, BUF>& sp, uint32_t e, const float* f) {
  if constexpr (BUF) {
    constexpr int N = Vec<T>::N;
    static_assert(W >= N, "the buffer path moves 16-byte vectors");
#pragma unroll
    for (int q = 0; q < W / N; ++q) sp.template store16<NT>(e + q * N, RawVec<T>::pack(f + q * N));
  } else {
    st<T, W, NT>(sp.p + e, f);
  }
}

template <typename T, int W, bool NT, bool BUF>
__device__ __forceinline__ void ld(const Span<T, BUF>& sp, uint32_t e, float* f) {
  if constexpr (BUF) {
    Frag<T, W> fr;
    fr.template load<NT>(sp, e);
    fr.unpack(f);
  } else {
    ld<T, W, NT>(sp.p + e, f);
  }
}

// ---------------------------------------------------------------------------
// Reductions.  Lane order and tree shape are fixed, so every reduction in this
// library is deterministic run to run (no floating-point atomics).
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sums NV per-thread values across a 256-thread workgroup.  The result is
// valid in thread 0 only (out[0..NV-1]).  `lds` must hold 4 * NV floats.
template <int NV>
__device__ __forceinline__ void block_sum(float (&v)[NV], float* lds) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = wave_sum(v[i]);
  if (lane == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) lds[wave * NV + i] = v[i];
  }
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = (lds[i] + lds[NV + i]) + (lds[2 * NV + i] + lds[3 * NV + i]);
  }
}

// ---------------------------------------------------------------------------
// Sums inside a 16-lane row of a wave with DPP (full-rate VALU, no LDS):
// quad-permute adds give the sum over a quad (sum_row16: lanes e ^ 1, e ^ 2),
// two row-rotate adds the sum over lanes e, e ^ 4, e ^ 8, e ^ 12 (sum_col16).
// Both trees add the same pairs in every lane, so all lanes that share a sum
// see bit-identical values.  All 16 lanes of a row must be active.  The
// Sinkhorn kernels use the pair as the row and column sums of a 4x4 matrix
// held one element per lane (lane e = 4 i + j).
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;  // row_ror:4
constexpr int kDppRowRor8 = 0x128;  // row_ror:8

// Sum over j of P[i][j] (the 4 lanes of a quad).
__device__ __forceinline__ float sum_row16(float v) {
  v += dpp<kDppQuadXor1>(v);
  return v + dpp<kDppQuadXor2>(v);
}

// Sum over i of P[i][j] (lanes e, e^4, e^8, e^12 of the 16-lane row).
__device__ __forceinline__ float sum_col16(float v) {
  v += dpp<kDppRowRor8>(v);
  return v + dpp<kDppRowRor4>(v);
}

__device__ __forceinline__ float sum_all16(float v) { return sum_col16(sum_row16(v)); }

// Sum of NV (<= 256) per-thread values over a 256-thread workgroup, for many
// values at once: each 16-lane row adds with DPP (sum_all16, full-rate VALU
// with no LDS crossbar traffic), the 16 row sums of each value go through LDS,
// and thread i < NV adds value i's row sums in row order.  Returns the total
// of value threadIdx.x in threads < NV.  A wave butterfly over __shfl_xor costs
// 6 ds_bpermute per value instead (600 for the weights projection's 100
// partials).
template <int NV>
__device__ __forceinline__ float block_sum_rows(float (&v)[NV], float* lds) {
  static_assert(NV <= kThreads, "one output per thread");
  const int row = threadIdx.x >> 4;
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] = sum_all16(v[i]);
  if ((threadIdx.x & 15) == 0) {
#pragma unroll
    for (int i = 0; i < NV; ++i) lds[row * NV + i] = v[i];
  }
  __syncthreads();
  float t = 0.f;
  if (threadIdx.x < NV) {
#pragma unroll
    for (int q = 0; q < kThreads / 16; ++q) t += lds[q * NV + threadIdx.x];
  }
  return t;
}

// block_sum for a workgroup of NT threads: one wave (the wave sum alone) or
// kThreads.  The result is valid in thread 0 only.  With one wave the result
// equals block_sum's whenever only the first wave holds non-zero values.
template <int NT, int NV>
__device__ __forceinline__ void group_sum(float (&v)[NV], float* lds) {
  static_assert(NT == 64 || NT == kThreads, "one wave or a full workgroup");
  if constexpr (NT == 64) {
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = wave_sum(v[i]);
  } else {
    block_sum<NV>(v, lds);
  }
}

// Zero-fills n floats.  A kernel rather than hipMemsetAsync so that callers may
// capture the work in a HIP graph.
template <int = 0>
__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// Host-side helpers shared by the entry points.
// ---------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* where);
int num_cus();

inline int fill_zero(float* p, int64_t n, hipStream_t st) {
  if (n <= 0) return MHC_OK;
  fill_zero_kernel<><<<dim3((unsigned)((n + 255) / 256)), 256, 0, st>>>(p, n);
  return hip_status(hipGetLastError(), "fill_zero launch");
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Batches go on grid.y; HIP caps grid.y, so larger batches are split into
// several launches by the entry points.
constexpr int64_t kMaxGridY = 65535;

}  // namespace mhc

// Dispatch on the bulk dtype: defines `using T = ...` inside the body.
#define MHC_DISPATCH_DTYPE(dtype, ...)                                   \
  [&]() -> int {                                                         \
    switch (dtype) {                                                     \
      case MHC_DTYPE_F32: { using T = float; return __VA_ARGS__(); }     \
      case MHC_DTYPE_BF16: { using T = __bf16; return __VA_ARGS__(); }   \
      case MHC_DTYPE_F16: { using T = _Float16; return __VA_ARGS__(); }  \
      default: ::mhc::set_error("unsupported dtype code %d", (int)(dtype)); \
               return MHC_ERR_DTYPE;                                     \
    }                                                                    \
  }()
