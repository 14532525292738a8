// Dynamic-weight kernels (Eq. 14-19) and the sequence mean-pool.
//
// Forward, standalone op (reference src/mhc/_kernels.py:318-590,690-752):
//   dynw_partial_kernel   split-K partial dot products x[r,:] . phi[:,j] (24)
//                         and sum(x^2) for a tile of RT rows and a K chunk,
//                         reading phi in its API layout [K,24]: one 96-byte
//                         row per k, contiguous across lanes (no transpose).
//   dynw_finalize_kernel  per row: fixed-order sum of the K-chunk partials,
//                         inv_rms, scale + bias, sigmoid / normalise, 2*sigmoid
//                         and the register-resident Sinkhorn of H_res
//                         (dynw_finalize_rows_kernel: the same for many rows
//                         with few K chunks, one 16-lane group per row).
// Layer path: colsum_reduce_kernel<PROJ=true> produces the same 25 partials
// per column chunk while it finishes the sequence mean, so the projection
// costs no extra pass over HBM.
//
// Backward (reference src/mhc/_kernels.py ops.py:110-228):
//   dynw_bwd_rows_kernel  per row: Sinkhorn backward, sigmoid / normalise
//                         backward, grad_raw, the rms coefficient and the
//                         per-row bias / alpha contributions.
//   dynw_bwd_wide_kernel  per k and row chunk: grad_x[r,k] = grad_raw[r,:] . phi[k,:]
//                         + coef[r] x[r,k] and grad_phi[k,:] = sum_r x[r,k] grad_raw[r,:]
//                         (per-chunk partials + dynw_gphi_reduce_kernel when
//                         rows are split).  Workgroup (0, 0) also sums
//                         grad_bias and grad_alpha over rows in a fixed order.
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
  __shared__ float lds[(kThreads / 16) * RT * kPart];
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
  const float tot = block_sum_rows<RT * kPart>(acc, lds);
  const int r = threadIdx.x / kPart, j = threadIdx.x - r * kPart;
  if (threadIdx.x < RT * kPart && r0 + r < R) part[((r0 + r) * nK + kc) * kPart + j] = tot;
}

// ---------------------------------------------------------------------------
// MFMA projection for many rows (the standalone op at R = tokens): the
// [R, K] x [K, 24] product on v_mfma_f32_32x32x16_bf16 (fp32 x is split
// exactly into three bf16 parts in registers; fp16 x goes through
// v_mfma_f32_32x32x16_f16 against a scaled two-part phi, below).  Fragment
// layout of these instructions (gfx950, checked on the device):
//   A: lane l, element j -> A[l % 32][8 (l / 32) + j]          (x rows)
//   B: lane l, element j -> B[8 (l / 32) + j][l % 32]          (phi columns)
//   D: lane l, element i -> D[8 (i / 4) + 4 (l / 32) + i % 4][l % 32]
// phi (fp32) is split into three bf16 parts, phi = hi + mid + lo +
// O(2^-27 |phi|), and all three are applied, so the projection keeps fp32
// accuracy (two parts leave 2^-18, which the 20-round Sinkhorn of H_res
// amplifies to ~1e-4 relative at K = 16384); columns 24..31 of B are zero.
// Each wave splits the phi values of its K slice into the three parts once,
// in registers, as the kernel starts (a separate packing kernel took 5 us at
// K = 16384).
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// a and b rounded to bf16 in one v_cvt_pk_bf16_f32 (a in the low half), and
// what that leaves of each, exactly: a = bf16(a) + ra.  Taking the rounded
// values back out of the packed word (a shift, a mask) keeps the compiler from
// converting each value again on its own to subtract it.
__device__ __forceinline__ uint32_t bf16_pair(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, bf16x2));
}
__device__ __forceinline__ uint32_t bf16_pair(float a, float b, float& ra, float& rb) {
  const uint32_t p = bf16_pair(a, b);
  ra = a - __uint_as_float(p << 16);
  rb = b - __uint_as_float(p & 0xffff0000u);
  return p;
}

// Forward projection on MFMA, K-slice form.  A workgroup of NW waves owns a
// K chunk of NW * S steps and a range of rows; wave w owns the chunk's steps
// w S .. w S + S - 1 (S * 32 bytes of each row) and keeps that slice's phi
// fragments (3 parts per step) in registers for the whole kernel, so phi costs
// no LDS or L2 traffic per x byte.  The workgroup walks its rows in 32-row
// tiles; per tile each wave loads its 32 rows x S * 32 bytes with 16-byte loads
// (S * 2 lanes per row), two tiles ahead, and passes them through its own LDS
// tile into the fragment layout (chunk c of row r in slot c ^ (r % (2 S))).
// At any time a workgroup streams NW * S * 32 = 2 KiB of each of 32 rows.  The
// row-owning form this replaces (waves owning 32 rows each, phi staged in LDS
// per 4-step group for a 512-row workgroup) streamed 128 bytes of each of 512
// rows: as a plain read, that pattern took 86 us at R = K = 16384 against 76
// for 512-byte runs, and the kernel took 108 us against 97 for this one.  The
// S * 3 MFMAs of a tile accumulate in one chain from zero (smallest part
// first); the NW waves' tile results and sums of squares meet in a
// double-buffered LDS area (one barrier per tile) and are added in wave order
// into 25-float partial records: part[r][kc][0:24] and the row's sum of
// squares [24], which the VALU forms from the A fragments alongside the MFMAs
// (v_dot2_f32_bf16 would take a quarter of the instructions, but its sums are
// not fp32-accurate: H_pre moved by 6e-3 relative at K = 4096).  Requires
// K % 16 == 0, a 16-byte aligned x, and rows_per_wg * K * sizeof(x) and
// K * 24 * 4 bytes under 2^31.
constexpr int kMfmaWaves = 8;                             // waves per workgroup (2 per SIMD)
constexpr int kMfmaSteps = 8;                             // 16-k steps per wave slice (16-bit x)
constexpr int kMfmaChunkSteps = kMfmaWaves * kMfmaSteps;  // steps per K chunk (16-bit x)
// fp32 x: half the steps per slice, so that a slice is still 256 bytes of a row
// and the LDS tiles keep their size
__host__ __device__ constexpr int mfma_steps(int esize) { return esize == 4 ? kMfmaSteps / 2 : kMfmaSteps; }
constexpr int kMfmaRedCols = kPart;                       // 24 dot products and the sum of squares
constexpr int kMfmaRedPitch = 36;                         // floats per (wave, column): 32 rows + pad

template <typename TX, int NW = kMfmaWaves, int S = mfma_steps(sizeof(TX))>
__global__ __launch_bounds__(64 * NW, 2) void dynw_mfma_kernel(const TX* __restrict__ x,
                                                             const float* __restrict__ phi,
                                                             float* __restrict__ part, int64_t R, int64_t K, int nK,
                                                             int64_t rows_per_wg) {
  constexpr int kThr = 64 * NW;
  constexpr int E = (int)sizeof(TX);
  constexpr int VE = 16 / E;     // elements per 16-byte chunk
  constexpr int CPF = 8 / VE;    // chunks per 8-element fragment
  constexpr int L = S * E;       // 16-byte chunks of a row in the wave's slice (S * 16 elements)
  constexpr int RPL = 64 / L;    // rows per load instruction
  constexpr int NL = 32 / RPL;   // loads per lane per tile
  static_assert(64 % L == 0 && 32 % RPL == 0, "slice shape");
  constexpr int kRedWave = kMfmaRedCols * kMfmaRedPitch;
  constexpr bool kXF16 = __is_same(TX, _Float16);
  constexpr bool kXF32 = __is_same(TX, float);
  static_assert(kXF16 || kXF32 || __is_same(TX, __bf16), "x is bf16, fp16 or fp32");
  __shared__ __attribute__((aligned(16))) u32x4 xt[NW][32 * L];
  __shared__ __attribute__((aligned(16))) float red[2][NW * kRedWave];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int kc = blockIdx.y;
  const int64_t nsteps = K / 16;
  const int64_t s0 = (int64_t)kc * (NW * S) + (int64_t)wave * S;  // the slice's first step
  int nvalid = (int)(nsteps - s0 < S ? nsteps - s0 : S);         // its steps inside K
  if (nvalid < 0) nvalid = 0;
  const int64_t rbeg = (int64_t)blockIdx.x * rows_per_wg;
  const int64_t rend = rbeg + rows_per_wg < R ? rbeg + rows_per_wg : R;
  if (rbeg >= rend) return;  // the whole workgroup
  // The slice's phi values, one fp32 per (step, element) and lane: lane l,
  // element j of step i -> phi[16 (s0 + i) + 8 (l / 32) + j][l % 32], through a
  // buffer span so that steps past K and columns 24..31 read zeros with no branch.
  const Span<float, true> phs(phi, K * kOut);
  uint32_t pv[S][8];
  {
    const int col = lane & 31;
    constexpr uint32_t kOobF32 = 0x20000000u;  // 2^31 bytes: past any span
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t k = 16 * (s0 + i) + 8 * (lane >> 5) + j;
        pv[i][j] = phs.load4<false>((i < nvalid && col < kOut) ? (uint32_t)(k * kOut + col) : kOobF32);
      }
  }
  u32x4 bf[S][3];  // filled below, while the first tiles' loads are in flight
  float unscale = 1.f;  // fp16 x: 1 / s of this lane's column (below)
  const int64_t ntile = (rend - rbeg + 31) / 32;
  const Span<TX, true> xs(x + rbeg * K, (rend - rbeg) * K);
  const int lr = lane / L, lc = lane % L;
  // element offset of load j of tile t: (32 t + RPL j + lr) K + 16 s0 + VE lc (past K: never used)
  const uint32_t lbase = (uint32_t)(lr * K + 16 * s0 + VE * lc);
  u32x4* tile = xt[wave];
  u32x4 a[2][NL];
  auto aload = [&](int64_t t, u32x4 (&d)[NL]) {
#pragma unroll
    for (int j = 0; j < NL; ++j) d[j] = xs.template load16<true>(lbase + (uint32_t)((32 * t + RPL * j) * K));
  };
  auto astage = [&](const u32x4 (&d)[NL]) {
#pragma unroll
    for (int j = 0; j < NL; ++j) {
      const int r = RPL * j + lr;
      tile[r * L + (lc ^ (r & (L - 1)))] = d[j];
    }
    // Lanes read what other lanes of the wave wrote: keep the order.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  const int fr = lane & 31, half = lane >> 5;
  // Tile t: its fragments from the wave's LDS tile, the chain, and the wave's
  // results into red[buf]; then the workgroup adds the NW records of each output.
  auto tile_compute = [&](int64_t t, int buf) {
    f32x16 st, st2;  // st2: the fp16 path's p2 products
#pragma unroll
    for (int i = 0; i < 16; ++i) st[i] = st2[i] = 0.f;
    float ss = 0.f, ss_hi = 0.f;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      if (i < nvalid) {
        const u32x4 d = tile[fr * L + ((CPF * (2 * i + half)) ^ (fr & (L - 1)))];
        const bf16x8 p_hi = __builtin_bit_cast(bf16x8, bf[i][0]);
        const bf16x8 p_mid = __builtin_bit_cast(bf16x8, bf[i][1]);
        const bf16x8 p_lo = __builtin_bit_cast(bf16x8, bf[i][2]);
        if constexpr (kXF32) {
          // fp32 x: each value splits exactly into bf16 hi + mid + lo (24 significant
          // bits, 8 per part).  Six products, smallest first; those below 2^-18 of
          // x phi (x_mid * phi_lo, x_lo * phi_mid, x_lo * phi_lo: 2^-27 and less,
          // the size of phi's own split residual) are dropped.
          const u32x4 d1 = tile[fr * L + ((CPF * (2 * i + half) + 1) ^ (fr & (L - 1)))];
          u32x4 ph, pm, pl;
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float a = __uint_as_float(c < 2 ? d[2 * c] : d1[2 * c - 4]);
            const float b = __uint_as_float(c < 2 ? d[2 * c + 1] : d1[2 * c - 3]);
            float ra, rb, la, lb;
            ph[c] = bf16_pair(a, b, ra, rb);    // ra, rb exact
            pm[c] = bf16_pair(ra, rb, la, lb);  // la, lb exact
            pl[c] = bf16_pair(la, lb);          // exact: at most 8 significant bits left
            ss = fmaf(a, a, ss);
            ss_hi = fmaf(b, b, ss_hi);
          }
          const bf16x8 xh = __builtin_bit_cast(bf16x8, ph);
          const bf16x8 xm = __builtin_bit_cast(bf16x8, pm);
          const bf16x8 xl = __builtin_bit_cast(bf16x8, pl);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, p_lo, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xm, p_mid, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, p_hi, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, p_mid, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xm, p_hi, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, p_hi, st, 0, 0, 0);
        } else if constexpr (kXF16) {
          // fp16 x: x as loaded against the two scaled fp16 parts of phi
          const f16x8 hv = __builtin_bit_cast(f16x8, d);
          st2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(hv, __builtin_bit_cast(f16x8, bf[i][1]), st2, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_f16(hv, __builtin_bit_cast(f16x8, bf[i][0]), st, 0, 0, 0);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float f = (float)hv[j];
            if (j & 1) ss_hi = fmaf(f, f, ss_hi);
            else ss = fmaf(f, f, ss);
          }
        } else {
          const bf16x8 av = __builtin_bit_cast(bf16x8, d);
          // smallest part first: the step sum sees the corrections before the bulk
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, p_lo, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, p_mid, st, 0, 0, 0);
          st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, p_hi, st, 0, 0, 0);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const float lo_ = __uint_as_float(d[c] << 16);
            const float hi_ = __uint_as_float(d[c] & 0xffff0000u);
            ss = fmaf(lo_, lo_, ss);
            ss_hi = fmaf(hi_, hi_, ss_hi);
          }
        }
      }
    }
    if constexpr (kXF16) {  // x (p1 + 2^-11 p2) / s, exact scalings
#pragma unroll
      for (int i = 0; i < 16; ++i) st[i] = fmaf(st2[i], 1.f / 2048.f, st[i]) * unscale;
    }
    float* rw = red[buf] + wave * kRedWave;
    // lane l holds column l % 32, rows 8 q + 4 (l / 32) + 0..3 in st[4 q .. 4 q + 3]
    if (fr < kOut) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
        *reinterpret_cast<f32x4*>(rw + fr * kMfmaRedPitch + 8 * q + 4 * half) =
            f32x4{st[4 * q], st[4 * q + 1], st[4 * q + 2], st[4 * q + 3]};
    }
    // the two k halves of a row's sum of squares sit in lanes l and l + 32
    const float sq = ss + ss_hi;
    const float sq2 = sq + __shfl_xor(sq, 32, 64);
    if (half == 0) rw[kOut * kMfmaRedPitch + fr] = sq2;
    __syncthreads();
    // output o of the tile: row o / 25, record entry o % 25 (consecutive threads
    // write one row's record); no branch between the NW reads
    const float* rb = red[buf];
#pragma unroll
    for (int q = 0; q < (32 * kPart + kThr - 1) / kThr; ++q) {
      const int o = threadIdx.x + q * kThr;
      if (o < 32 * kPart) {
        const int row = o / kPart, c = o - row * kPart;
        const int64_t r = rbeg + 32 * t + row;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += rb[w * kRedWave + c * kMfmaRedPitch + row];
        if (r < rend) part[(r * nK + kc) * kPart + c] = v;
      }
    }
  };
  // Tile t's loads sit in a[t % 2]; the loop is unrolled by two so that
  // neither register set is copied, and runs an even number of tiles.  Every
  // path issues the same loads: a tile past the end lies past the span and
  // reads zeros without touching memory, and writes no records.  (With the
  // next tile's loads behind a branch, or a mid-loop exit, the compiler's wait
  // before a tile's staging has to hold for a path that skipped them, and
  // waits for the loads in flight as well: 23 us more at R = K = 16384.)  The
  // other waves read red[buf] of tile t until they reach the barrier of tile
  // t + 1, so tile t + 2 may write it.
  aload(0, a[0]);
  __builtin_amdgcn_sched_barrier(0);  // tile 0's loads first: the first wait is for them alone
  aload(1, a[1]);
  __builtin_amdgcn_sched_barrier(0);
  // phi in three bf16 parts, phi = hi + mid + lo + O(2^-27 |phi|), while the
  // first two tiles' loads are in flight.  fp16 x instead: the f16 MFMA takes x
  // as it is, and phi goes in as two fp16 parts of its column scaled by a power
  // of two, s phi = p1 + 2^-11 p2 + O(2^-22 |s phi|), with s chosen per wave
  // slice and column so that the column's largest |s phi| lies in [2^14, 2^15)
  // (no fp16 overflow); the two products accumulate apart and meet, unscaled,
  // at the end of each tile.
  if constexpr (kXF16) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < S; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) mx = fmaxf(mx, fabsf(__uint_as_float(pv[i][j])));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));  // lanes l and l + 32 hold one column
    mx = fminf(mx, 0x1.fffffep127f);          // an infinite phi gets a finite exponent (and NaN products)
    int ex = 0;
    if (mx > 0.f) frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
    // s = 2^(15 - ex), held to 2^126 so that s and 1 / s stay finite and normal
    // (a column below 2^-111 then scales into [2^-112, 2^15), still fp16 normals
    // down to 2^-126 of its largest entry)
    const int es = mx > 0.f ? min(15 - ex, 126) : 0;
    const float sc = ldexpf(1.f, es);
    unscale = ldexpf(1.f, -es);
#pragma unroll
    for (int i = 0; i < S; ++i) {
      f16x8 p1, p2;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = __uint_as_float(pv[i][j]) * sc;  // exact
        const _Float16 h = (_Float16)v;
        p1[j] = h;
        p2[j] = (_Float16)((v - (float)h) * 2048.f);  // v - h exact
      }
      bf[i][0] = __builtin_bit_cast(u32x4, p1);
      bf[i][1] = __builtin_bit_cast(u32x4, p2);
    }
  } else {
#pragma unroll
  for (int i = 0; i < S; ++i) {
    bf16x8 hi, mid, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = __uint_as_float(pv[i][j]);
      const __bf16 h = (__bf16)v;
      const float r1 = v - (float)h;  // exact in fp32
      const __bf16 m = (__bf16)r1;
      hi[j] = h;
      mid[j] = m;
      lo[j] = (__bf16)(r1 - (float)m);
    }
    bf[i][0] = __builtin_bit_cast(u32x4, hi);
    bf[i][1] = __builtin_bit_cast(u32x4, mid);
    bf[i][2] = __builtin_bit_cast(u32x4, lo);
  }
  }
  for (int64_t t = 0; t < ntile; t += 2) {
    astage(a[0]);
    aload(t + 2, a[0]);
    tile_compute(t, 0);
    astage(a[1]);
    aload(t + 3, a[1]);
    tile_compute(t + 1, 1);
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

// Eq. 14-19 epilogue of one row in 16-lane form: lane e owns H_res element e;
// lanes 0..3 also H_pre[e], lanes 4..7 H_post[e - 4].  raw_res = raw[8 + e],
// raw_pp = raw[e & 7] and sumsq (the row's sum of x^2) are the row's totals.
// All 16 lanes of the row must take part (DPP sums); lanes with !store
// compute and write nothing.
__device__ __forceinline__ void finalize_row16(int e, int64_t r, float raw_res, float raw_pp, float sumsq,
                                               int64_t K, const DynParams& P, OutRow o_pre, OutRow o_post,
                                               OutRow o_res, float* __restrict__ aux, int iters, float eps,
                                               bool store) {
  const int j = e & 3;
  const bool is_pre = e < 4;
  const float inv_rms = 1.f / sqrtf(sumsq / (float)K + eps);
  // Eq. 19: H_res = Sinkhorn(|s_res| + eps)
  const float m = sk16_forward(inv_rms * *P.alpha_res * raw_res + P.bias_res[e], iters, eps);
  // Eq. 17: H_pre = sigmoid / (sum + eps); Eq. 18: H_post = 2 sigmoid
  const float s_pp = inv_rms * (is_pre ? *P.alpha_pre : *P.alpha_post) * raw_pp +
                     (is_pre ? P.bias_pre[j] : P.bias_post[j]);
  const float sg = sigmoidf(s_pp);
  const float den = sum_row16(sg) + eps;  // quad 0: the four H_pre sigmoids
  if (!store) return;
  o_res.p[r * o_res.stride + e] = m;
  if (is_pre) o_pre.p[r * o_pre.stride + j] = sg / den;
  else if (e < 8) o_post.p[r * o_post.stride + j] = 2.f * sg;
  if (aux) {
    aux[r * kPart + 8 + e] = raw_res;
    if (e < 8) aux[r * kPart + e] = raw_pp;
    if (e == 0) aux[r * kPart + kOut] = inv_rms;
  }
}

// One wave per row.  Lane l sums the partial records l, l+64, l+128, ... (25
// floats each) in chunk order; each 16-lane row of the wave then adds its lane
// sums with DPP (sum_all16), and lanes 0..15 add the four row sums in order
// and run the epilogue.  Keeping 64 independent load streams per row instead
// of one serial chain matters: R is the batch (4 at dim 4096) and this kernel
// sits between two full passes over H.  (A __shfl_xor butterfly took 150
// ds_bpermute per wave for the same sums.)
template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_finalize_kernel(const float* __restrict__ part, int nK, int64_t R,
                                                                 int64_t K, DynParams P, OutRow o_pre,
                                                                 OutRow o_post, OutRow o_res,
                                                                 float* __restrict__ aux, int iters, float eps) {
  __shared__ float quarter[4][4][kPart];  // [wave][16-lane row][value]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + wave;
  const bool live = r < R;
  float acc[kPart];
#pragma unroll
  for (int j = 0; j < kPart; ++j) acc[j] = 0.f;
  for (int k = lane; live && k < nK; k += 64) {
    const float* p = part + (r * nK + k) * kPart;
#pragma unroll
    for (int j = 0; j < kPart; ++j) acc[j] += p[j];
  }
#pragma unroll
  for (int j = 0; j < kPart; ++j) acc[j] = sum_all16(acc[j]);
  if ((lane & 15) == 0) {
#pragma unroll
    for (int j = 0; j < kPart; ++j) quarter[wave][lane >> 4][j] = acc[j];
  }
  __syncthreads();
  if (!live || lane >= 16) return;
  const float(*q)[kPart] = quarter[wave];
  auto tot = [&](int j) { return ((q[0][j] + q[1][j]) + q[2][j]) + q[3][j]; };
  finalize_row16(lane, r, tot(8 + lane), tot(lane & 7), tot(kOut), K, P, o_pre, o_post, o_res, aux, iters, eps,
                 true);
}

// The same for many rows with few chunks (the MFMA projection at R = tokens:
// R = 16384, nK = 16): one 16-lane group per row, 16 rows per workgroup.  Lane
// e sums, in chunk order, only the three record entries its epilogue reads
// (raw[8 + e], raw[e & 7] and the sum of squares), so no cross-lane reduction
// is needed.  One wave per row left three quarters of each wave idle in the
// epilogue and spent 25 butterflies per row (33 us at R = 16384).
constexpr int kFinRowsWg = 16;

template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_finalize_rows_kernel(const float* __restrict__ part, int nK,
                                                                      int64_t R, int64_t K, DynParams P,
                                                                      OutRow o_pre, OutRow o_post, OutRow o_res,
                                                                      float* __restrict__ aux, int iters,
                                                                      float eps) {
  const int e = threadIdx.x & 15;
  const int64_t r_grp = (int64_t)blockIdx.x * kFinRowsWg + (threadIdx.x >> 4);
  const bool live = r_grp < R;
  const int64_t r = live ? r_grp : R - 1;  // idle groups redo the last row and store nothing
  const float* p = part + r * nK * kPart;
  float raw_res = 0.f, raw_pp = 0.f, sumsq = 0.f;
  // unrolled so that the chunks' loads are in flight together (the sums keep
  // chunk order): 8.4 us at R = 16384, nK = 16, against 10.9 us rolled and
  // 15.2 us unrolled by 16
#pragma unroll 8
  for (int k = 0; k < nK; ++k, p += kPart) {
    raw_res += p[8 + e];
    raw_pp += p[e & 7];
    sumsq += p[kOut];
  }
  finalize_row16(e, r, raw_res, raw_pp, sumsq, K, P, o_pre, o_post, o_res, aux, iters, eps, live);
}

// Per-row backward record rowbuf[r][0:52]:
//   [0:24]  grad_raw  = g_scaled * inv_rms * alpha_g
//   [24]    coef      : grad_x += coef * x  (rms path)
//   [25:49] g_scaled  (-> grad_bias)
//   [49:52] per-group sum g_scaled * inv_rms * raw (-> grad_alpha)
// Follows reference src/mhc/ops.py:138-216 with the Sinkhorn part of
// _backward.py:30-262 (sgn(0) = 0).
//
// RPW rows per 256-thread workgroup (R is the batch in the layer path, so
// this is a latency problem).  In the layer path the upstream H_pre / H_res
// gradients arrive as the weight-gradient pass's per-workgroup partials
// part20[r][k][0:20] (4 H_pre, 16 H_res) over nblk workgroups, which the
// workgroup sums itself: with RPW = 4, wave w sums row w's partials; with
// RPW = 1 (the layer path, up to 2048 partials per row at B = 1) all four
// waves share the row and their sums are added in wave order.  Lanes stride
// the chunks with 16-byte loads, then a fixed butterfly.  The standalone op
// passes the gradients as rows (g_pre [R,4], g_res [R,16]).  Wave 0 then runs
// the rows in 16-lane form: lane e of a group owns H_res element e, lanes 0..3
// also H_pre[e], lanes 4..7 H_post[e - 4].
constexpr int kSkSlots = 32;  // Sinkhorn states kept in LDS per lane

template <int RPW>
__global__ __launch_bounds__(kThreads) void dynw_bwd_rows_kernel(const float* __restrict__ aux, DynParams P,
                                                                 InRow h_pre, InRow g_pre, InRow g_post,
                                                                 InRow g_res, const float* __restrict__ part20,
                                                                 int nblk, float* __restrict__ rowbuf, int64_t R,
                                                                 int64_t K, int iters, float eps) {
  static_assert(RPW == 1 || RPW == 4 || RPW == 16, "rows per workgroup");
  // RPW = 16 (gradients as rows only, no part20): every wave runs four rows.
  constexpr int kRowWaves = RPW == 16 ? 4 : 1;
  __shared__ float slots[kSkSlots * 64 * kRowWaves];
  __shared__ float red[4][20];
  __shared__ float quarter[4][4][20];  // [wave][16-lane row][value]
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  if (RPW != 16 && part20) {
    const int64_t rw = (int64_t)blockIdx.x * RPW + (RPW == 4 ? wave : 0);
    const int k0 = RPW == 4 ? lane : wave * 64 + lane;
    const int kstep = RPW == 4 ? 64 : 256;
    f32x4 acc[5];
#pragma unroll
    for (int q = 0; q < 5; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (rw < R) {
#pragma unroll 4
      for (int k = k0; k < nblk; k += kstep) {
        const f32x4* p = reinterpret_cast<const f32x4*>(part20 + (rw * nblk + k) * 20);
#pragma unroll
        for (int q = 0; q < 5; ++q) acc[q] += p[q];
      }
    }
    // Each 16-lane row adds its lane sums with DPP; the row sums then add in
    // order through LDS (per wave with RPW == 4, over the workgroup with 1).
#pragma unroll
    for (int q = 0; q < 5; ++q) {
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float v = sum_all16(acc[q][c]);
        if ((lane & 15) == 0) quarter[wave][lane >> 4][4 * q + c] = v;
      }
    }
    __syncthreads();
    if (RPW == 1) {
      if (threadIdx.x < 20) {
        const int v = threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w)
#pragma unroll
          for (int h = 0; h < 4; ++h) t += quarter[w][h][v];
        red[0][v] = t;
      }
    } else if (lane < 20) {
      red[wave][lane] = ((quarter[wave][0][lane] + quarter[wave][1][lane]) + quarter[wave][2][lane]) +
                        quarter[wave][3][lane];
    }
  }
  if constexpr (RPW != 16) {
    __syncthreads();
    if (wave != 0) return;
  }
  const int e = lane & 15;
  const int j = e & 3;
  const int64_t r_grp = (int64_t)blockIdx.x * RPW + (RPW == 16 ? 4 * wave : 0) + (lane >> 4);
  const bool live = r_grp < R && (RPW == 16 || (lane >> 4) < RPW);
  const int64_t r = live ? r_grp : R - 1;  // idle groups redo the last row and store nothing
  const int rr = RPW == 4 ? (lane >> 4) : 0;  // this group's row in `red`
  const bool from_part = RPW != 16 && part20;
  const float gpre = from_part ? red[rr][j] : (g_pre.p ? g_pre.p[r * g_pre.stride + j] : 0.f);
  const float gres = from_part ? red[rr][4 + e] : (g_res.p ? g_res.p[r * g_res.stride + e] : 0.f);
  const float gpost = g_post.p ? g_post.p[r * g_post.stride + j] : 0.f;
  const float* a = aux + r * kPart;
  const float inv_rms = a[kOut];
  const float ar = *P.alpha_res;
  const float raw_res = a[8 + e];
  const float raw_pp = a[e & 7];
  // H_res = Sinkhorn(|s_res| + eps): gradient w.r.t. s_res.
  const float s_res = inv_rms * ar * raw_res + P.bias_res[e];
  const float gs_res = iters == 20 ? sk16_backward_fixed<20>(s_res, gres, eps)
                                   : sk16_backward<kSkSlots>(s_res, gres, iters, eps,
                                                             slots + (RPW == 16 ? wave * kSkSlots * 64 : 0) + lane, 64);
  // H_pre = sigmoid / (sum + eps) on lanes 0..3, H_post = 2 sigmoid on lanes 4..7.
  const bool is_pre = (e & 4) == 0;
  const float al_pp = is_pre ? *P.alpha_pre : *P.alpha_post;
  const float sg = sigmoidf(inv_rms * al_pp * raw_pp + (is_pre ? P.bias_pre[j] : P.bias_post[j]));
  const float hp = h_pre.p[r * h_pre.stride + j];
  const float den = sum_row16(sg) + eps;   // quad 0: sum of the H_pre sigmoids
  const float dot = sum_row16(gpre * hp);  // quad 0: <g_pre, H_pre>
  const float gs_pp = is_pre ? (gpre - dot) / den * sg * (1.f - sg) : gpost * 2.f * sg * (1.f - sg);
  const bool has_pp = e < 8;
  // Group sums for grad_alpha and the rms path.
  const float ga_res = sum_all16(gs_res * inv_rms * raw_res);
  const float ga_pp = sum_row16(has_pp ? gs_pp * inv_rms * raw_pp : 0.f);  // lane 0: pre, lane 4: post
  const float g_inv = sum_all16(gs_res * ar * raw_res + (has_pp ? gs_pp * al_pp * raw_pp : 0.f));
  if (!live) return;
  float* rb = rowbuf + r * kRow;
  rb[8 + e] = gs_res * inv_rms * ar;
  rb[33 + e] = gs_res;
  if (has_pp) {
    rb[e] = gs_pp * inv_rms * al_pp;
    rb[25 + e] = gs_pp;
  }
  // inv_rms = 1/rms, rms = sqrt(sum x^2 / K + eps): d rms / d x = x / (K rms)
  if (e == 0) {
    rb[24] = g_inv * (-inv_rms * inv_rms) * inv_rms / (float)K;
    rb[49] = ga_pp;
    rb[51] = ga_res;
  }
  if (e == 4) rb[50] = ga_pp;
}

// Thread per k over the rows of one row chunk (grid.y):
//   grad_x[r,k] = grad_raw[r,:] . phi[k,:] + coef[r] x[r,k]   (written as TG)
//   grad_phi[k,:] (+)= sum_{r in chunk} x[r,k] grad_raw[r,:]
// With one row chunk grad_phi is written directly; otherwise each chunk
// writes gphi_part[chunk][k][0:24] and dynw_gphi_reduce_kernel sums the
// chunks in order.  The per-row record is the same for every thread of the
// workgroup (scalar loads).  With grad_bias or grad_alpha requested, the
// launcher adds one column of workgroups, whose workgroup (last, 0) sums the
// per-row records into grad_bias [24] and grad_alpha [3] (threads stride over
// rows, then a fixed-order block sum) alongside the others instead of ahead
// of its own columns; the rows' x loads are issued four at a time (at the
// layer's R = 4: 4.8 against 7.2 us).  launch_dynw_bwd_wide picks one-wave workgroups
// (kWideThreads = 64) when R <= 64: the work is then a few loads and ~50 FMAs
// per k, so the pass is latency-bound and wants every CU busy -- at the
// layer's R = 4, K = 16384, 256 one-wave workgroups take 3.1 us against 6.6 us
// for 64 of 256 threads, with the same results.  With more rows it keeps 256
// threads, so that workgroup (0, 0)'s walk over the rows stays short.
constexpr int kWideThreads = 64;

template <typename TX, typename TG, int NT = kThreads>
__global__ __launch_bounds__(NT) void dynw_bwd_wide_kernel(const TX* __restrict__ x,
                                                                 const float* __restrict__ phi,
                                                                 const float* __restrict__ rowbuf,
                                                                 TG* __restrict__ gx, float* __restrict__ gphi,
                                                                 float* __restrict__ gphi_part,
                                                                 float* __restrict__ gbias,
                                                                 float* __restrict__ galpha, int64_t R, int64_t K,
                                                                 int64_t RC, bool phi_vec) {
  if ((gbias || galpha) && blockIdx.x == gridDim.x - 1) {
    // the launcher's extra column of workgroups: (last, 0) sums the records, the rest have no work
    if (blockIdx.y != 0) return;
    __shared__ float lds[4 * 27];
    float acc[27];
#pragma unroll
    for (int i = 0; i < 27; ++i) acc[i] = 0.f;
    for (int64_t r = threadIdx.x; r < R; r += NT) {
      const float* rb = rowbuf + r * kRow;
#pragma unroll
      for (int i = 0; i < 27; ++i) acc[i] += rb[25 + i];
    }
    group_sum<NT, 27>(acc, lds);
    if (threadIdx.x == 0) {
#pragma unroll
      for (int j = 0; j < kOut; ++j) if (gbias) gbias[j] = acc[j];
#pragma unroll
      for (int g = 0; g < 3; ++g) if (galpha) galpha[g] = acc[24 + g];
    }
    return;
  }
  const int64_t k = (int64_t)blockIdx.x * NT + threadIdx.x;
  if (k >= K || (!gx && !gphi)) return;
  const int64_t r_beg = (int64_t)blockIdx.y * RC;
  const int64_t r_end = r_beg + RC < R ? r_beg + RC : R;
  float ph[kOut], gp[kOut];
  load_phi_row(phi, k, phi_vec, ph);
#pragma unroll
  for (int j = 0; j < kOut; ++j) gp[j] = 0.f;
  // four rows at a time, their x loads issued together
  for (int64_t r0 = r_beg; r0 < r_end; r0 += 4) {
    float xq[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) xq[q] = r0 + q < r_end ? to_f32(x[(r0 + q) * K + k]) : 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (r0 + q < r_end) {
        const int64_t r = r0 + q;
        const float* rb = rowbuf + r * kRow;
        const float xv = xq[q];
        float v = rb[24] * xv;
#pragma unroll
        for (int j = 0; j < kOut; ++j) {
          v += rb[j] * ph[j];
          gp[j] += xv * rb[j];
        }
        if (gx) gx[r * K + k] = from_f32<TG>(v);
      }
    }
  }
  float* o = gphi_part ? gphi_part + ((int64_t)blockIdx.y * K + k) * kOut : gphi;
  if (o) {
#pragma unroll
    for (int j = 0; j < kOut; ++j) o[(gphi_part ? 0 : k * kOut) + j] = gp[j];
  }
}

template <typename TX, typename TG>
inline hipError_t launch_dynw_bwd_wide(const TX* x, const float* phi, const float* rowbuf, TG* gx, float* gphi,
                                       float* gphi_part, float* gbias, float* galpha, int64_t R, int64_t K,
                                       int64_t RC, unsigned nR, bool phi_vec, hipStream_t st) {
  if (R <= kWideThreads) {
    const unsigned ncol = (K > 0 ? (unsigned)((K + kWideThreads - 1) / kWideThreads) : 1u) + (gbias || galpha ? 1u : 0u);
    dynw_bwd_wide_kernel<TX, TG, kWideThreads><<<dim3(ncol, nR), kWideThreads, 0, st>>>(
        x, phi, rowbuf, gx, gphi, gphi_part, gbias, galpha, R, K, RC, phi_vec);
  } else {
    const unsigned ncol = (K > 0 ? (unsigned)((K + kThreads - 1) / kThreads) : 1u) + (gbias || galpha ? 1u : 0u);
    dynw_bwd_wide_kernel<TX, TG, kThreads><<<dim3(ncol, nR), kThreads, 0, st>>>(
        x, phi, rowbuf, gx, gphi, gphi_part, gbias, galpha, R, K, RC, phi_vec);
  }
  return hipGetLastError();
}

// The wide pass for many rows (the standalone op at R = tokens), both products
// on MFMA (v_mfma_f32_32x32x16_bf16; fragment layout above; fp16 x is split
// exactly into bf16 hi + lo for grad_phi, fp32 x into hi + mid):
//   grad_x [R, K]  = G [R, 24] phi^T [24, K] + coef [R] x      (x's dtype out)
//   grad_phi [K, 24] = x^T [K, R] G [R, 24]                      (f32, per chunk)
// with G = grad_raw = rowbuf[r][0:24] and coef = rowbuf[r][24].  A workgroup
// of kBwdWaves waves owns kBwdCols = 32 * kBwdWaves columns (wave w: the
// 32-column block at 32 w) and a chunk of RC rows, walked in 64-row blocks.
// The x strip a workgroup reads and the grad_x strip it writes are 512 bytes
// of each row: as a plain copy, 256-byte strips (128 columns, four waves)
// peak at 67% of 8 TB/s and 512-byte strips at 79%, at the same grid size.
// Per block the x tile (bf16) and the G rows are staged in LDS, with the next
// kBwdAhead = 2 blocks' loads in flight (streaming loads and stores: x is read and
// grad_x written once).  G is split into bf16 hi + lo planes once, as it is
// staged (fp32 products then take hi*hi + hi*lo + lo*hi, relative error ~2^-16):
//   grad_x: computed transposed, grad_x^T = phi G^T, so that the A operand is
//           the wave's phi fragments (registers for the whole kernel) and
//           the B operand 16-byte reads of the G planes.  Each lane then holds
//           one row and four runs of four consecutive columns: the epilogue
//           adds coef * x with 8-byte LDS reads and writes bf16 to an LDS tile
//           with 8-byte writes, and the tile leaves as coalesced 16-byte
//           stores (8-byte stores straight from registers were 30% slower);
//   grad_phi: A = x^T and B = G from the LDS tiles by transpose reads
//           (ds_read_b64_tr_b16: within each 16-lane group, lane i receives
//           element i % 4 of the 8 bytes lane 4 j + i / 4 addresses, j = 0..3),
//           accumulated in the MFMA registers over the chunk, and read ahead
//           of the grad_x work; the two 32-row halves' grad_x chains run
//           interleaved.
// The LDS padding leaves 2-way bank conflicts on the transpose and epilogue
// reads; making those reads conflict-free (wrong results, timing only) saved
// 1%.  At R = K = 16384 the kernel takes about 181 us with 4 row chunks of
// 4096 rows (one workgroup per CU), 200 us with 16 chunks of 1024; with 16
// chunks, copies of it without the grad_x stores took 168 us and without the
// MFMA work 181 us, against 170 us for a plain copy of the same strips
// (1024 workgroups).  Requires K a multiple of 16 bytes of x (8 elements of
// 16-bit x, 4 of fp32) and 16-byte aligned x and grad_x.  Grid (K / kBwdCols column blocks, row
// chunks); outputs as dynw_bwd_wide_kernel: grad_phi direct with one chunk,
// else per-chunk partials.  Column block 0 of each row chunk also sums the
// chunk's grad_bias / grad_alpha records after its main loop: into gbias /
// galpha with one chunk, else into bias_part[chunk][27], which
// dynw_gphi_reduce_kernel adds in chunk order.
constexpr int kBwdWaves = 8;              // waves per workgroup (32 columns each)
constexpr int kBwdMinWaves = 2;           // waves per SIMD the register allocation must allow
constexpr int kBwdRows = 64;              // rows per staged block (two 32-row MFMA halves)
constexpr int kBwdAhead = 2;              // blocks of loads in flight: register sets (three: slower)
constexpr int kBwdGPitch = 40;            // bf16 per LDS row of the split G planes (columns 24..31 zero)

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// 64-bit LDS transpose read of 16-bit elements (see above).
__device__ __forceinline__ u32x2 lds_read_tr16(const __bf16* p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p)));
}

template <typename TX, typename TG = TX, int AH = (sizeof(TX) == 4 || sizeof(TG) == 4) ? 1 : kBwdAhead,
          int NW = kBwdWaves, int MINW = kBwdMinWaves>
__global__ __launch_bounds__(64 * NW, MINW) void dynw_bwd_mfma_kernel(const TX* __restrict__ x,
                                                                    const float* __restrict__ phi,
                                                                    const float* __restrict__ rowbuf,
                                                                    TG* __restrict__ gx, float* __restrict__ gphi,
                                                                    float* __restrict__ gphi_part,
                                                                    float* __restrict__ bias_part,
                                                                    float* __restrict__ gbias,
                                                                    float* __restrict__ galpha, int64_t R, int64_t K,
                                                                    int64_t RC) {
  constexpr int kBwdThreads = 64 * NW;
  constexpr int kBwdCols = 32 * NW;            // columns per workgroup
  constexpr int E = (int)sizeof(TX);
  constexpr int VE = 16 / E;                   // x elements per 16-byte vector
  constexpr int kBwdXPitch = kBwdCols + VE;    // elements per padded LDS row of the x / grad_x tiles
  constexpr int TR = kBwdRows;
  constexpr int XLPR = kBwdCols / VE;          // lanes per x row (16 bytes each)
  constexpr int XRPP = kBwdThreads / XLPR;     // x rows per pass of the workgroup
  constexpr int NX = TR / XRPP;                // 16-byte x vectors per lane per block
  // grad_x is written in TG: x's type, or f32 from 16-bit x (the layer at S = 1 reads H's rows
  // as x and keeps grad_x in f32 for pass C); same tile walk with TG's vector width
  constexpr int EG = (int)sizeof(TG);
  constexpr int VEG = 16 / EG;
  constexpr int kBwdGXPitch = kBwdCols + VEG;  // elements per padded LDS row of the grad_x tile
  constexpr int XLPRG = kBwdCols / VEG;
  constexpr int XRPPG = kBwdThreads / XLPRG;
  constexpr int NXG = TR / XRPPG;
  static_assert(TR % XRPPG == 0 && (__is_same(TG, TX) || __is_same(TG, float)), "grad_x tile");
  constexpr int GRPP = kBwdThreads / 8;        // G rows per pass (8 lanes per 32-float row)
  constexpr int NG = TR / GRPP > 0 ? TR / GRPP : 1;
  static_assert(TR % XRPP == 0 && (TR % GRPP == 0 || GRPP >= TR), "block shape");
  constexpr bool kXF16 = __is_same(TX, _Float16);
  constexpr bool kXF32 = __is_same(TX, float);
  static_assert(kXF16 || kXF32 || __is_same(TX, __bf16), "x is bf16, fp16 or fp32");
  // Blocks of loads in flight (AH): by default one for fp32 x, whose blocks are twice the bytes in
  // the same registers, and for an f32 grad_x from 16-bit x (layer backward at S = 1, D = 4096:
  // 32.2 -> 30.0 us at 64 rows, the same at 1024 and 4096 rows), else kBwdAhead; the launcher
  // takes one for chunks of a single block.
  constexpr int A = AH;
  static_assert(A >= 1 && A <= kBwdAhead, "blocks ahead");
  // The x and grad_x tiles hold TX and TG values (fp32: 2 x 66.5 KiB of LDS); the G planes are bf16.
  __shared__ __attribute__((aligned(16))) TX xs[TR * kBwdXPitch];
  __shared__ __attribute__((aligned(16))) TG gxs[TR * kBwdGXPitch];
  __shared__ __attribute__((aligned(16))) __bf16 ghi[TR * kBwdGPitch];
  __shared__ __attribute__((aligned(16))) __bf16 glo[TR * kBwdGPitch];
  __shared__ float cf[TR];
  const int64_t r_beg = (int64_t)blockIdx.y * RC;
  const int64_t r_end = r_beg + RC < R ? r_beg + RC : R;
  // grad_bias and grad_alpha: the rows' records 25..51 summed over the rows.  Column block 0
  // sums its row chunk after its main loop (below): with one chunk into gbias / galpha, else
  // into bias_part[chunk] for dynw_gphi_reduce_kernel.  (One workgroup summing all 16384 rows
  // of R = K = 16384 before its main loop finished ~70 us after the others.)
  const bool do_bias = blockIdx.x == 0 && (bias_part || gbias || galpha);
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t k0 = (int64_t)blockIdx.x * kBwdCols;
  // phi fragments: lane l, element e -> phi[k0 + 32 wave + l % 32][16 js + 8 (l / 32) + e].
  bf16x8 bhi[2], blo[2];
  {
    const int64_t kk = k0 + 32 * wave + (lane & 31);
#pragma unroll
    for (int js = 0; js < 2; ++js) {
      const int j0 = 16 * js + 8 * (lane >> 5);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float v = (kk < K && j0 + e < kOut) ? phi[kk * kOut + j0 + e] : 0.f;
        const __bf16 h = (__bf16)v;
        bhi[js][e] = h;
        blo[js][e] = (__bf16)(v - (float)h);
      }
    }
  }
  // Tile loads: x rows t / XLPR + XRPP i (16 bytes at column 8 (t % XLPR)); G record row
  // t / 8 + GRPP j, floats 4 (t % 8)..+3.  x, grad_x and the G records go through buffer
  // spans of the chunk's rows, so that every load and store is issued on every path: rows
  // past the chunk read zeros and drop their stores, and lanes without a column use an
  // offset past any span.  (Loads and stores behind branches made the compiler's wait
  // before each block's staging hold for a path without them, so it waited for the next
  // block's loads as well.)
  const int64_t nrows = r_end - r_beg;
  const Span<TX, true> xsp(x + r_beg * K, nrows * K);
  const Span<TG, true> gxsp(gx ? gx + r_beg * K : reinterpret_cast<const TG*>(x), gx ? nrows * K : 0);
  const Span<float, true> gsp(rowbuf + r_beg * kRow, nrows * kRow);
  constexpr uint32_t kOobX = 0x80000000u / E, kOobG = 0x80000000u / EG, kOobF32 = 0x20000000u;  // 2^31 bytes
  const int xr = threadIdx.x / XLPR;
  const int xc = (threadIdx.x % XLPR) * VE;
  const bool xcol_ok = k0 + xc < K;
  const int grow = threadIdx.x >> 3;
  const int gcol = (threadIdx.x & 7) * 4;
  const bool g_ok = grow < TR;
  const bool gld_ok = g_ok && gcol < 28;
  // element offsets in the spans of row i of this lane in block b
  auto xoff = [&](int64_t b, int i) -> uint32_t {
    return xcol_ok ? (uint32_t)((TR * b + xr + XRPP * i) * K + k0 + xc) : kOobX;
  };
  const int gxr = threadIdx.x / XLPRG;
  const int gxc = (threadIdx.x % XLPRG) * VEG;
  const bool gxcol_ok = k0 + gxc < K;
  auto goff = [&](int64_t b, int i) -> uint32_t {
    return gxcol_ok ? (uint32_t)((TR * b + gxr + XRPPG * i) * K + k0 + gxc) : kOobG;
  };
  auto load_block = [&](int64_t b, u32x4 (&xv)[NX], f32x4 (&gv)[NG]) {
#pragma unroll
    for (int i = 0; i < NX; ++i) xv[i] = xsp.template load16<true>(xoff(b, i));
#pragma unroll
    for (int j = 0; j < NG; ++j)
      gv[j] = __builtin_bit_cast(
          f32x4, gsp.load16<false>(gld_ok ? (uint32_t)((TR * b + grow + GRPP * j) * kRow + gcol) : kOobF32));
  };
  // Transpose-read addresses: 16-lane group gi = lane / 16 covers columns 16 (gi & 1) .. +15 of
  // the wave's 32 and rows 8 (gi >> 1) + 0..3 of a 16-row step (+4 for the second read).
  const int gi = lane >> 4, l16 = lane & 15;
  const int tr_row = 8 * (gi >> 1) + (l16 >> 2);
  const int tr_col = 16 * (gi & 1) + 4 * (l16 & 3);
  f32x16 zero, dphi;
#pragma unroll
  for (int i = 0; i < 16; ++i) zero[i] = 0.f;
  dphi = zero;
  // One 64-row block b of the chunk: stage the registers loaded for it, refill them with the
  // block two ahead, compute, write its grad_x tile.
  auto block = [&](int64_t b, u32x4 (&xv)[NX], f32x4 (&gv)[NG]) {
    // Stage this block: x as loaded, G split into hi + lo planes, coef apart.
#pragma unroll
    for (int i = 0; i < NX; ++i) *reinterpret_cast<u32x4*>(&xs[(xr + XRPP * i) * kBwdXPitch + xc]) = xv[i];
    if (g_ok) {
#pragma unroll
      for (int jj = 0; jj < NG; ++jj) {
        const int gr = grow + GRPP * jj;
        u32x2 h4, l4;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          float ra, rb;
          h4[c] = bf16_pair(gcol < kOut ? gv[jj][2 * c] : 0.f, gcol < kOut ? gv[jj][2 * c + 1] : 0.f, ra, rb);
          l4[c] = bf16_pair(ra, rb);
        }
        *reinterpret_cast<u32x2*>(&ghi[gr * kBwdGPitch + gcol]) = h4;
        *reinterpret_cast<u32x2*>(&glo[gr * kBwdGPitch + gcol]) = l4;
        if (gcol == kOut) cf[gr] = gv[jj][0];
      }
    }
    __syncthreads();
    load_block(b + A, xv, gv);  // in flight during the compute below
    // grad_phi operands for the block's 16-row steps, read before the grad_x work so that their
    // LDS latency overlaps it.  A = x^T (lane l: column 32 wave + l % 32, rows
    // 16 st + 8 (l / 32) + e), B = G (same rows, j = l % 32).  16-bit x comes through the
    // transpose read; fp32 x as eight 4-byte reads per step (consecutive lanes, consecutive
    // columns).
    constexpr int NST = TR / 16;
    bf16x8 pa[NST], pbh[NST], pbl[NST];
    float pa32[kXF32 ? NST : 1][8];
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      const int rb = 16 * st + tr_row;
      if constexpr (kXF32) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pa32[st][e] = xs[(16 * st + 8 * (lane >> 5) + e) * kBwdXPitch + 32 * wave + (lane & 31)];
      } else {
        const u32x2 x0 = lds_read_tr16(reinterpret_cast<const __bf16*>(&xs[rb * kBwdXPitch + 32 * wave + tr_col]));
        const u32x2 x1 =
            lds_read_tr16(reinterpret_cast<const __bf16*>(&xs[(rb + 4) * kBwdXPitch + 32 * wave + tr_col]));
        pa[st] = __builtin_bit_cast(bf16x8, u32x4{x0[0], x0[1], x1[0], x1[1]});
      }
      const u32x2 h0 = lds_read_tr16(&ghi[rb * kBwdGPitch + tr_col]);
      const u32x2 h1 = lds_read_tr16(&ghi[(rb + 4) * kBwdGPitch + tr_col]);
      const u32x2 q0 = lds_read_tr16(&glo[rb * kBwdGPitch + tr_col]);
      const u32x2 q1 = lds_read_tr16(&glo[(rb + 4) * kBwdGPitch + tr_col]);
      pbh[st] = __builtin_bit_cast(bf16x8, u32x4{h0[0], h0[1], h1[0], h1[1]});
      pbl[st] = __builtin_bit_cast(bf16x8, u32x4{q0[0], q0[1], q1[0], q1[1]});
    }
    // grad_x^T = phi G^T (see above) for the two 32-row halves as two independent chains,
    // interleaved; each chain takes its products smallest first, hi x hi last.
    constexpr int NH = TR / 32;
    bf16x8 ghv[NH][2], glv[NH][2];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh)
#pragma unroll
      for (int js = 0; js < 2; ++js) {
        const int j0 = 16 * js + 8 * (lane >> 5);
        ghv[hh][js] = *reinterpret_cast<const bf16x8*>(&ghi[(32 * hh + (lane & 31)) * kBwdGPitch + j0]);
        glv[hh][js] = *reinterpret_cast<const bf16x8*>(&glo[(32 * hh + (lane & 31)) * kBwdGPitch + j0]);
      }
    f32x16 d[NH];
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) d[hh] = zero;
#pragma unroll
    for (int js = 0; js < 2; ++js) {
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) d[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bhi[js], glv[hh][js], d[hh], 0, 0, 0);
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) d[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(blo[js], ghv[hh][js], d[hh], 0, 0, 0);
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) d[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bhi[js], ghv[hh][js], d[hh], 0, 0, 0);
    }
    // grad_phi += x^T G over the steps (one chain, in step order).  fp16 x splits exactly
    // into bf16 hi + lo (|lo| <= 2^-9 |x|); x_lo * G_lo (2^-18 of x G, the size of G's own
    // split residual) is dropped.
#pragma unroll
    for (int st = 0; st < NST; ++st) {
      if constexpr (kXF32) {
        // fp32 x: bf16 hi + mid parts (x_lo * G_hi and x_mid * G_lo, 2^-18 of x G, are dropped
        // as above)
        u32x4 ph, pm;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float ra, rb;
          ph[c] = bf16_pair(pa32[st][2 * c], pa32[st][2 * c + 1], ra, rb);
          pm[c] = bf16_pair(ra, rb);
        }
        const bf16x8 xh = __builtin_bit_cast(bf16x8, ph);
        const bf16x8 xm = __builtin_bit_cast(bf16x8, pm);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, pbl[st], dphi, 0, 0, 0);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xm, pbh[st], dphi, 0, 0, 0);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, pbh[st], dphi, 0, 0, 0);
      } else if constexpr (kXF16) {
        const f16x8 hv = __builtin_bit_cast(f16x8, pa[st]);
        u32x4 ph, pl;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float ra, rb;
          ph[c] = bf16_pair((float)hv[2 * c], (float)hv[2 * c + 1], ra, rb);
          pl[c] = bf16_pair(ra, rb);  // exact
        }
        const bf16x8 xh = __builtin_bit_cast(bf16x8, ph);
        const bf16x8 xl = __builtin_bit_cast(bf16x8, pl);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, pbl[st], dphi, 0, 0, 0);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xl, pbh[st], dphi, 0, 0, 0);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xh, pbh[st], dphi, 0, 0, 0);
      } else {
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[st], pbl[st], dphi, 0, 0, 0);
        dphi = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[st], pbh[st], dphi, 0, 0, 0);
      }
    }
    // Epilogue: lane l holds row l % 32 of its half, columns 32 wave + 8 q + 4 (l / 32) + 0..3
    // in d[hh][4 q ..].
#pragma unroll
    for (int hh = 0; hh < NH; ++hh) {
      const int row = 32 * hh + (lane & 31);
      const float c = cf[row];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int cc = 32 * wave + 8 * q + 4 * (lane >> 5);
        typedef TX tx4 __attribute__((ext_vector_type(4)));
        typedef TG tg4 __attribute__((ext_vector_type(4)));
        const tx4 x4 = *reinterpret_cast<const tx4*>(&xs[row * kBwdXPitch + cc]);
        tg4 o4;
#pragma unroll
        for (int r = 0; r < 4; ++r) o4[r] = (TG)(d[hh][4 * q + r] + c * (float)x4[r]);
        *reinterpret_cast<tg4*>(&gxs[row * kBwdGXPitch + cc]) = o4;
      }
    }
    __syncthreads();
    // grad_x tile out: rows gxr + XRPPG i, 16 bytes at column gxc (no grad_x: an empty span).
#pragma unroll
    for (int i = 0; i < NXG; ++i)
      gxsp.template store16<true>(goff(b, i),
                                  *reinterpret_cast<const u32x4*>(&gxs[(gxr + XRPPG * i) * kBwdGXPitch + gxc]));
    // No barrier here: every read of xs / ghi / glo / cf in this block came
    // before the barrier above, and gxs is next written after the next
    // block's first barrier, which waits for these reads.
  };
  // Blocks rotate through A register sets, each refilled with the block A ahead; the loop
  // runs a multiple of A blocks (those past the chunk read zeros and store nothing).
  u32x4 xv[A][NX];
  f32x4 gv[A][NG];
  const int64_t nblk = (nrows + TR - 1) / TR;
#pragma unroll
  for (int u = 0; u < A; ++u) {
    load_block(u, xv[u], gv[u]);
    __builtin_amdgcn_sched_barrier(0);  // in block order: each wait is for the oldest loads alone
  }
  for (int64_t b = 0; b < nblk; b += A) {
#pragma unroll
    for (int u = 0; u < A; ++u) block(b + u, xv[u], gv[u]);
  }
  if (do_bias) {
    // this chunk's rows strided over the workgroup's threads, then the wave sums in wave order
    __shared__ float lds[NW * 27];
    float acc[27];
#pragma unroll
    for (int i = 0; i < 27; ++i) acc[i] = 0.f;
    for (int64_t r = r_beg + threadIdx.x; r < r_end; r += kBwdThreads) {
      const float* rb = rowbuf + r * kRow;
#pragma unroll
      for (int i = 0; i < 27; ++i) acc[i] += rb[25 + i];
    }
#pragma unroll
    for (int i = 0; i < 27; ++i) acc[i] = wave_sum(acc[i]);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 27; ++i) lds[wave * 27 + i] = acc[i];
    }
    __syncthreads();
    if (threadIdx.x < 27) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) t += lds[w * 27 + threadIdx.x];
      if (bias_part) bias_part[(int64_t)blockIdx.y * 27 + threadIdx.x] = t;
      else if (threadIdx.x < kOut) { if (gbias) gbias[threadIdx.x] = t; }
      else if (galpha) galpha[threadIdx.x - kOut] = t;
    }
  }
  // grad_phi: lane l, element i -> k = k0 + 32 wave + 8 (i / 4) + 4 (l / 32) + i % 4, j = l % 32.
  const int j = lane & 31;
  float* o = gphi_part ? gphi_part + (int64_t)blockIdx.y * K * kOut : gphi;
  if (j >= kOut || !o) return;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int64_t kk = k0 + 32 * wave + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
    if (kk < K) o[kk * kOut + j] = dphi[i];
  }
}

// grad_phi[i] = sum over row chunks c (in order) of gphi_part[c][i], i < n = K * 24
// (n = 0: no grad_phi), and, with bias_part given, grad_bias / grad_alpha from
// the chunks' 27-float records, in threads n .. n + 26.
template <int = 0>
__global__ __launch_bounds__(kThreads) void dynw_gphi_reduce_kernel(const float* __restrict__ part,
                                                                    float* __restrict__ gphi, int64_t n, int nc,
                                                                    const float* __restrict__ bias_part,
                                                                    float* __restrict__ gbias,
                                                                    float* __restrict__ galpha) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i < n) {
    float v = 0.f;
#pragma unroll 4
    for (int c = 0; c < nc; ++c) v += part[(int64_t)c * n + i];
    gphi[i] = v;
  } else if (bias_part && i < n + 27) {
    const int j = (int)(i - n);
    float v = 0.f;
    for (int c = 0; c < nc; ++c) v += bias_part[c * 27 + j];
    if (j < kOut) { if (gbias) gbias[j] = v; }
    else if (galpha) galpha[j - kOut] = v;
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
// Loads go through a buffer span rebased at each group of UN rows (the host
// keeps UN rows of K under 2^31 bytes).  The first nt_rows rows of each S
// chunk are read with the streaming (nt) policy, the rest plain: what
// branch_input reads next and can find in the 256 MB memory-side cache is the
// tail of every chunk, and nt on the rest speeds this read up.
template <bool NT, typename T, int W, int UN, bool BUF>
__device__ __forceinline__ void colsum_rows(const T* base, int64_t K, uint32_t lane_e, int64_t& s, int64_t end,
                                            float* acc) {
  for (; s + (UN - 1) < end; s += UN) {
    const Span<T, BUF> sp(base + s * K, (int64_t)UN * K);
    float v[UN][W];
#pragma unroll
    for (int u = 0; u < UN; ++u) ld<T, W, NT>(sp, (uint32_t)(u * K) + lane_e, v[u]);
#pragma unroll
    for (int u = 0; u < UN; ++u)
#pragma unroll
      for (int e = 0; e < W; ++e) acc[e] += v[u][e];
  }
  for (; s < end; ++s) {
    const Span<T, BUF> sp(base + s * K, K);
    float v[W];
    ld<T, W, NT>(sp, lane_e, v);
#pragma unroll
    for (int e = 0; e < W; ++e) acc[e] += v[e];
  }
}

template <typename T, int W, int UN, bool BUF = (W > 1)>
__global__ __launch_bounds__(kThreads) void colsum_kernel(const T* __restrict__ H, float* __restrict__ colpart,
                                                          int64_t S, int64_t K, int64_t SC, int nS, int64_t nt_rows,
                                                          int64_t b0) {
  const int64_t b = b0 + blockIdx.z;
  const int sc = blockIdx.y;
  const int64_t cblk = (int64_t)blockIdx.x * (kThreads * W);
  const int64_t col = cblk + (int64_t)threadIdx.x * W;
  if (col >= K) return;
  const int64_t sbeg = (int64_t)sc * SC;
  const int64_t send = sbeg + SC < S ? sbeg + SC : S;
  const int64_t smid = sbeg + nt_rows < send ? sbeg + nt_rows : send;
  float acc[W];
#pragma unroll
  for (int e = 0; e < W; ++e) acc[e] = 0.f;
  const T* base = H + b * S * K + cblk;
  const uint32_t lane_e = (uint32_t)threadIdx.x * W;
  int64_t s = sbeg;
  colsum_rows<true, T, W, UN, BUF>(base, K, lane_e, s, smid, acc);
  colsum_rows<false, T, W, UN, BUF>(base, K, lane_e, s, send, acc);
  st<float, W>(colpart + ((b * nS + sc) * K + col), acc);
}

template <bool PROJ>
__global__ __launch_bounds__(kThreads) void colsum_reduce_kernel(const float* __restrict__ colpart,
                                                                 float* __restrict__ x,
                                                                 const float* __restrict__ phi,
                                                                 float* __restrict__ projpart, int64_t K, int nS,
                                                                 float inv_S, int64_t b0, bool phi_vec) {
  __shared__ float red[(kThreads / 16) * kPart];
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
    if (x) x[b * K + c] = v;  // with the projection x is optional (nothing reads it after a no-grad forward)
    if constexpr (PROJ) {
      float ph[kOut];
      load_phi_row(phi, c, phi_vec, ph);
#pragma unroll
      for (int j = 0; j < kOut; ++j) pv[j] = v * ph[j];
      pv[kOut] = v * v;
    }
  }
  if constexpr (PROJ) {
    const float tot = block_sum_rows<kPart>(pv, red);
    if (threadIdx.x < kPart) projpart[(b * gridDim.x + blockIdx.x) * kPart + threadIdx.x] = tot;
  }
}

// Short sequences (the decode regime): the two kernels above in one launch.
// One thread per column sums H[b, s, c] over the same S chunks of SC rows, in
// the same order, as colsum_kernel and colsum_reduce_kernel do (each chunk from
// zero, then the chunk sums in chunk order, then the 1/S scale), so x and the
// projection partials come out bit for bit as on the two-kernel path; what
// goes is the column-partial round trip and one dependent launch.
template <typename T, bool PROJ>
__global__ __launch_bounds__(kThreads) void colsum_direct_kernel(const T* __restrict__ H, float* __restrict__ x,
                                                                 const float* __restrict__ phi,
                                                                 float* __restrict__ projpart, int64_t S, int64_t K,
                                                                 int64_t SC, float inv_S, int64_t b0, bool phi_vec) {
  __shared__ float red[(kThreads / 16) * kPart];
  const int64_t b = b0 + blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  float pv[kPart];
#pragma unroll
  for (int j = 0; j < kPart; ++j) pv[j] = 0.f;
  if (c < K) {
    const T* p = H + b * S * K + c;
    float v = 0.f;
    for (int64_t s0 = 0; s0 < S; s0 += SC) {
      const int64_t s1 = s0 + SC < S ? s0 + SC : S;
      float a = 0.f;
#pragma unroll 4
      for (int64_t s = s0; s < s1; ++s) a += to_f32(p[s * K]);
      v += a;
    }
    v *= inv_S;
    if (x) x[b * K + c] = v;  // with the projection x is optional (nothing reads it after a no-grad forward)
    if constexpr (PROJ) {
      float ph[kOut];
      load_phi_row(phi, c, phi_vec, ph);
#pragma unroll
      for (int j = 0; j < kOut; ++j) pv[j] = v * ph[j];
      pv[kOut] = v * v;
    }
  }
  if constexpr (PROJ) {
    const float tot = block_sum_rows<kPart>(pv, red);
    if (threadIdx.x < kPart) projpart[(b * gridDim.x + blockIdx.x) * kPart + threadIdx.x] = tot;
  }
}

// The same without the projection, W columns per lane through 16-byte loads (a
// workgroup per 256 W columns of a batch instead of per 256: at B = 4096, S = 1,
// D = 4096 the one-column form launched 262,144 workgroups); the per-column sums
// are the same operations, so the bits are too.
template <typename T, int W>
__global__ __launch_bounds__(kThreads) void colsum_direct_vec_kernel(const T* __restrict__ H, float* __restrict__ x,
                                                                     int64_t S, int64_t K, int64_t SC, float inv_S,
                                                                     int64_t b0) {
  const int64_t b = b0 + blockIdx.y;
  const int64_t c = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * W;
  if (c >= K) return;
  const T* p = H + b * S * K + c;
  float v[W];
#pragma unroll
  for (int e = 0; e < W; ++e) v[e] = 0.f;
  for (int64_t s0 = 0; s0 < S; s0 += SC) {
    const int64_t s1 = s0 + SC < S ? s0 + SC : S;
    float a[W];
#pragma unroll
    for (int e = 0; e < W; ++e) a[e] = 0.f;
#pragma unroll 4
    for (int64_t s = s0; s < s1; ++s) {
      float f[W];
      ld<T, W>(p + s * K, f);
#pragma unroll
      for (int e = 0; e < W; ++e) a[e] += f[e];
    }
#pragma unroll
    for (int e = 0; e < W; ++e) v[e] += a[e];
  }
#pragma unroll
  for (int e = 0; e < W; ++e) v[e] *= inv_S;
  st<float, W>(x + b * K + c, v);
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
