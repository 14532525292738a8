// Access-pattern ceilings of the two MFMA dynamic-weights kernels (the
// standalone fused_dynamic_weights op at R = tokens): how fast can a kernel
// with the same grid, the same per-lane loads and stores, the same register
// pipeline and the same LDS reservation move x (and grad_x) when it does none
// of the arithmetic?  Not part of the C ABI of the mHC path (libmhc_hip.so);
// built into libmhc_probe.so and loaded only by `bench.py --dynw-ceiling`.
//
// Forward (dynw_mfma_kernel's pattern): grid (row ranges, K chunks), 8 waves;
// wave w streams 32 rows x 256 bytes of its K slice per tile, two tiles of
// loads in flight in two register sets.  Modes add the kernel's costs one at a
// time, so the differences split the kernel's time:
//   0  loads only (each lane folds its vectors into one live value)
//   1  + staging: the vectors go through the wave's LDS tile (XOR-swizzled, as
//        the kernel lays them out) and come back in fragment order
//   2  + one workgroup barrier per tile
//   3  + the split-K records: 32 rows x 25 floats per tile and K chunk
//   4  as 3 with the records chunk-major and stored as 16-byte vectors
// Backward (dynw_bwd_mfma_kernel's pattern): grid (256-column blocks, row
// chunks), 8 waves; each workgroup walks its rows in 64-row blocks of
// 512-byte strips, two blocks of loads in flight:
//   0  read only
//   1  copy: each loaded vector is stored to the same place of grad_x
//   2  copy through LDS: the block staged in an x tile, a barrier, copied to a
//        grad_x tile, a barrier, stored from there (the kernel's two
//        barriers per block and its tile traffic)
//   3  as 2 with the tiles doubled by block parity: each pair of blocks stores
//        both grad_x tiles after the second block's barrier (64-KiB store
//        bursts per workgroup, three barriers per pair)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../dynw_kernels.hpp"

namespace {

using mhc::Span;
using mhc::u32x4;

constexpr int kFwdWaves = mhc::kMfmaWaves;
constexpr int kFwdSteps = mhc::kMfmaSteps;
constexpr int kFwdThreads = 64 * kFwdWaves;
constexpr int kL = 2 * kFwdSteps;  // 16-byte chunks of a row in a wave's slice
constexpr int kRPL = 64 / kL;      // rows per load instruction
constexpr int kNL = 32 / kRPL;     // loads per lane per tile

template <int MODE>
__global__ __launch_bounds__(kFwdThreads, 2) void dynw_fwd_pattern_kernel(const __bf16* __restrict__ x,
                                                                          float* __restrict__ part, int64_t R,
                                                                          int64_t K, int nK, int64_t rows_per_wg,
                                                                          unsigned* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) u32x4 lds[];  // sized like the kernel's tiles and records
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int kc = blockIdx.y;
  const int64_t s0 = (int64_t)kc * (kFwdWaves * kFwdSteps) + (int64_t)wave * kFwdSteps;
  const int64_t rbeg = (int64_t)blockIdx.x * rows_per_wg;
  const int64_t rend = rbeg + rows_per_wg < R ? rbeg + rows_per_wg : R;
  if (rbeg >= rend) return;
  const int64_t ntile = (rend - rbeg + 31) / 32;
  const Span<__bf16, true> xs(x + rbeg * K, (rend - rbeg) * K);
  const int lr = lane / kL, lc = lane % kL;
  const uint32_t lbase = (uint32_t)(lr * K + 16 * s0 + 8 * lc);
  u32x4* tile = lds + wave * (32 * kL);
  const int fr = lane & 31, half = lane >> 5;
  u32x4 a[2][kNL];
  u32x4 acc = u32x4{0u, 0u, 0u, 0u};
  auto aload = [&](int64_t t, u32x4 (&d)[kNL]) {
#pragma unroll
    for (int j = 0; j < kNL; ++j) d[j] = xs.load16<true>(lbase + (uint32_t)((32 * t + kRPL * j) * K));
  };
  auto consume = [&](int64_t t, u32x4 (&d)[kNL]) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int j = 0; j < kNL; ++j) acc ^= d[j];
    } else {
#pragma unroll
      for (int j = 0; j < kNL; ++j) {
        const int r = kRPL * j + lr;
        tile[r * kL + (lc ^ (r & (kL - 1)))] = d[j];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int i = 0; i < kFwdSteps; ++i) acc ^= tile[fr * kL + ((2 * i + half) ^ (fr & (kL - 1)))];
      if constexpr (MODE >= 2) __syncthreads();
      if constexpr (MODE == 3) {
        const float v = (float)(acc.x & 0xffu);
#pragma unroll
        for (int q = 0; q < (32 * mhc::kPart + kFwdThreads - 1) / kFwdThreads; ++q) {
          const int o = threadIdx.x + q * kFwdThreads;
          if (o < 32 * mhc::kPart) {
            const int row = o / mhc::kPart, c = o - row * mhc::kPart;
            const int64_t r = rbeg + 32 * t + row;
            if (r < rend) part[(r * nK + kc) * mhc::kPart + c] = v;
          }
        }
      } else if constexpr (MODE == 4) {
        // the same records chunk-major ([chunk][row][25]: a tile's 32 records are 800
        // consecutive floats), each of 200 threads storing 16 bytes
        const float v = (float)(acc.x & 0xffu);
        constexpr int kVec = 32 * mhc::kPart / 4;
        if (threadIdx.x < kVec) {
          const int64_t r0 = rbeg + 32 * t;
          const int64_t nrec = rend - r0 < 32 ? rend - r0 : 32;
          if (4 * threadIdx.x + 4 <= nrec * mhc::kPart)  // whole vectors inside the range only
            *reinterpret_cast<mhc::f32x4*>(part + ((int64_t)kc * R + r0) * mhc::kPart + 4 * threadIdx.x) =
                mhc::f32x4{v, v, v, v};
        }
      }
    }
  };
  aload(0, a[0]);
  __builtin_amdgcn_sched_barrier(0);
  aload(1, a[1]);
  __builtin_amdgcn_sched_barrier(0);
  for (int64_t t = 0; t < ntile; t += 2) {
    consume(t, a[0]);
    aload(t + 2, a[0]);
    consume(t + 1, a[1]);
    aload(t + 3, a[1]);
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == acc.w) sink[threadIdx.x & 255] = acc.x;
}

constexpr int kBwdWaves = mhc::kBwdWaves;
constexpr int kBwdThreads = 64 * kBwdWaves;
constexpr int kBwdCols = 32 * kBwdWaves;
constexpr int kBwdPitch = kBwdCols + 8;          // bf16 per padded LDS row, as in the kernel
constexpr int kTR = mhc::kBwdRows;               // rows per block
constexpr int kXLPR = kBwdCols / 8;              // lanes per row (16 bytes each)
constexpr int kXRPP = kBwdThreads / kXLPR;       // rows per pass
constexpr int kNX = kTR / kXRPP;                 // vectors per lane per block
constexpr int kAhead = mhc::kBwdAhead;

template <int MODE>
__global__ __launch_bounds__(kBwdThreads, mhc::kBwdMinWaves) void dynw_bwd_pattern_kernel(
    const __bf16* __restrict__ x, __bf16* __restrict__ gx, int64_t R, int64_t K, int64_t RC,
    unsigned* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) __bf16 tiles[];  // x tile, grad_x tile, the kernel's G planes
  __bf16* xt = tiles;
  __bf16* gt = tiles + kTR * kBwdPitch;
  const int64_t r_beg = (int64_t)blockIdx.y * RC;
  const int64_t r_end = r_beg + RC < R ? r_beg + RC : R;
  const int64_t nrows = r_end - r_beg;
  const int64_t k0 = (int64_t)blockIdx.x * kBwdCols;
  const Span<__bf16, true> xsp(x + r_beg * K, nrows * K);
  const Span<__bf16, true> gxsp(gx + r_beg * K, MODE == 0 ? 0 : nrows * K);
  constexpr uint32_t kOob = 0x40000000u;
  const int xr = threadIdx.x / kXLPR;
  const int xc = (threadIdx.x % kXLPR) * 8;
  const bool col_ok = k0 + xc < K;
  auto off = [&](int64_t b, int i) -> uint32_t {
    return col_ok ? (uint32_t)((kTR * b + xr + kXRPP * i) * K + k0 + xc) : kOob;
  };
  u32x4 acc = u32x4{0u, 0u, 0u, 0u};
  u32x4 xv[kAhead][kNX];
  auto load_block = [&](int64_t b, u32x4 (&v)[kNX]) {
#pragma unroll
    for (int i = 0; i < kNX; ++i) v[i] = xsp.load16<true>(off(b, i));
  };
  auto block = [&](int64_t b, u32x4 (&v)[kNX]) {
    if constexpr (MODE == 0) {
#pragma unroll
      for (int i = 0; i < kNX; ++i) acc ^= v[i];
      load_block(b + kAhead, v);
    } else if constexpr (MODE == 1) {
      u32x4 o[kNX];
#pragma unroll
      for (int i = 0; i < kNX; ++i) o[i] = v[i] ^ u32x4{1u, 0u, 0u, 0u};
      load_block(b + kAhead, v);
#pragma unroll
      for (int i = 0; i < kNX; ++i) gxsp.store16<true>(off(b, i), o[i]);
    } else if constexpr (MODE == 3) {
      // two x tiles and two grad_x tiles by block parity; the second block of each pair stores
      // both blocks' grad_x tiles after its barrier (64-KiB bursts, three barriers per pair)
      const int par = (int)(b & 1);
      __bf16* xp = xt + par * (2 * kTR * kBwdPitch);
      __bf16* gp = gt + par * (2 * kTR * kBwdPitch);
#pragma unroll
      for (int i = 0; i < kNX; ++i) *reinterpret_cast<u32x4*>(&xp[(xr + kXRPP * i) * kBwdPitch + xc]) = v[i];
      __syncthreads();
      load_block(b + kAhead, v);
      const int yr = (xr + 1) % kXRPP;
#pragma unroll
      for (int i = 0; i < kNX; ++i)
        *reinterpret_cast<u32x4*>(&gp[(yr + kXRPP * i) * kBwdPitch + xc]) =
            *reinterpret_cast<const u32x4*>(&xp[(yr + kXRPP * i) * kBwdPitch + xc]);
      if (par) {
        __syncthreads();
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const __bf16* gq = gt + q * (2 * kTR * kBwdPitch);
#pragma unroll
          for (int i = 0; i < kNX; ++i)
            gxsp.store16<true>(off(b - 1 + q, i), *reinterpret_cast<const u32x4*>(&gq[(xr + kXRPP * i) * kBwdPitch + xc]));
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < kNX; ++i) *reinterpret_cast<u32x4*>(&xt[(xr + kXRPP * i) * kBwdPitch + xc]) = v[i];
      __syncthreads();
      load_block(b + kAhead, v);
      // each lane copies another lane's 16 bytes, so the tile's contents cross lanes
      const int yr = (xr + 1) % kXRPP;
#pragma unroll
      for (int i = 0; i < kNX; ++i)
        *reinterpret_cast<u32x4*>(&gt[(yr + kXRPP * i) * kBwdPitch + xc]) =
            *reinterpret_cast<const u32x4*>(&xt[(yr + kXRPP * i) * kBwdPitch + xc]);
      __syncthreads();
#pragma unroll
      for (int i = 0; i < kNX; ++i)
        gxsp.store16<true>(off(b, i), *reinterpret_cast<const u32x4*>(&gt[(xr + kXRPP * i) * kBwdPitch + xc]));
    }
  };
  const int64_t nblk = (nrows + kTR - 1) / kTR;
#pragma unroll
  for (int u = 0; u < kAhead; ++u) {
    load_block(u, xv[u]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int64_t b = 0; b < nblk; b += kAhead) {
#pragma unroll
    for (int u = 0; u < kAhead; ++u) block(b + u, xv[u]);
  }
  if (acc.x == 0x9e3779b9u && acc.y == 0x7f4a7c15u && acc.z == acc.w) sink[threadIdx.x & 255] = acc.x;
}

// LDS of the real kernels, reserved dynamically so the probes run at the same occupancy.
constexpr size_t kFwdLds = sizeof(u32x4) * kFwdWaves * 32 * kL +
                           sizeof(float) * 2 * kFwdWaves * mhc::kMfmaRedCols * mhc::kMfmaRedPitch;
constexpr size_t kBwdLds = sizeof(__bf16) * (2 * kTR * kBwdPitch + 2 * kTR * mhc::kBwdGPitch) + sizeof(float) * kTR;
// mode 3: two x and two grad_x tiles (the x tile of parity p at p * 2 tiles, its grad_x tile after it)
constexpr size_t kBwdLds3 = kBwdLds + sizeof(__bf16) * 2 * kTR * kBwdPitch;

}  // namespace

// Forward pattern over x [R, K] bf16 with mode 0..3 (above), the kernel's plan:
// nK chunks of kFwdWaves * kFwdSteps * 16 columns, row ranges of rows_per_wg;
// `part` holds R * nK * 25 floats (mode 3).  Backward pattern over x and
// grad_x [R, K] bf16 with mode 0..3 and row chunks of RC rows.  `sink` is 1 KiB
// of device memory that keeps loaded values live.  Returns 0, 1 for a bad
// argument, 2 for a launch error.
extern "C" int mhc_probe_dynw(int pattern, int mode, const void* x, void* out, int64_t R, int64_t K,
                              int64_t rows, void* sink, void* stream) {
  if (!x || !sink || R <= 0 || K <= 0 || K % 16 != 0 || rows <= 0) return 1;
  if (rows * K * 2 >= ((int64_t)1 << 31)) return 1;
  hipStream_t st = (hipStream_t)stream;
  unsigned* s = (unsigned*)sink;
  if (pattern == 0) {
    const int nK = (int)((K / 16 + kFwdWaves * kFwdSteps - 1) / (kFwdWaves * kFwdSteps));
    if (mode >= 3 && !out) return 1;
    const dim3 grid((unsigned)((R + rows - 1) / rows), (unsigned)nK);
    const __bf16* xb = (const __bf16*)x;
    float* p = (float*)out;
    switch (mode) {
      case 0: dynw_fwd_pattern_kernel<0><<<grid, kFwdThreads, kFwdLds, st>>>(xb, p, R, K, nK, rows, s); break;
      case 1: dynw_fwd_pattern_kernel<1><<<grid, kFwdThreads, kFwdLds, st>>>(xb, p, R, K, nK, rows, s); break;
      case 2: dynw_fwd_pattern_kernel<2><<<grid, kFwdThreads, kFwdLds, st>>>(xb, p, R, K, nK, rows, s); break;
      case 3: dynw_fwd_pattern_kernel<3><<<grid, kFwdThreads, kFwdLds, st>>>(xb, p, R, K, nK, rows, s); break;
      case 4: dynw_fwd_pattern_kernel<4><<<grid, kFwdThreads, kFwdLds, st>>>(xb, p, R, K, nK, rows, s); break;
      default: return 1;
    }
  } else if (pattern == 1) {
    if (K % kBwdCols != 0 || (mode > 0 && !out)) return 1;
    const dim3 grid((unsigned)(K / kBwdCols), (unsigned)((R + rows - 1) / rows));
    const __bf16* xb = (const __bf16*)x;
    __bf16* g = (__bf16*)out;
    switch (mode) {
      case 0: dynw_bwd_pattern_kernel<0><<<grid, kBwdThreads, kBwdLds, st>>>(xb, g, R, K, rows, s); break;
      case 1: dynw_bwd_pattern_kernel<1><<<grid, kBwdThreads, kBwdLds, st>>>(xb, g, R, K, rows, s); break;
      case 2: dynw_bwd_pattern_kernel<2><<<grid, kBwdThreads, kBwdLds, st>>>(xb, g, R, K, rows, s); break;
      case 3: dynw_bwd_pattern_kernel<3><<<grid, kBwdThreads, kBwdLds3, st>>>(xb, g, R, K, rows, s); break;
      default: return 1;
    }
  } else {
    return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
