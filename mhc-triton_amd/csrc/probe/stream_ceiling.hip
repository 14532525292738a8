// Streaming-ceiling probe: how fast can a kernel shaped like the layer's
// streaming kernels move a given mix of reads and writes on this GPU?  Not part
// of the C ABI of the mHC path (libmhc_hip.so); built into libmhc_probe.so and
// loaded only by `bench.py --stream-ceiling`.
//
// The tensors are laid out like the layer's: per token, an input array holds
// NA (resp. NB, NC) rows of `row_bytes` and the output array NW rows, token
// after token ([T, rows, D] row-major).  One workgroup of 256 lanes owns one
// tile = (token, 4 KiB column block) when rows are whole tiles, else 256
// consecutive flattened items; each lane moves one 16-byte vector per
// row through a buffer resource, as the layer kernels do, with every load of
// the tile issued before the first use.  Output row w is the 32-bit sum of
// all input rows plus one of them; with no output the sum is kept live by a
// store that never fires.
// The occupancy cap (workgroups per CU) is set with a dynamic-LDS reservation,
// as in the layer kernels.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../stream_kernels.hpp"

namespace {

using mhc::Span;
using mhc::u32x4;

constexpr int kLanes = 256;
constexpr int kTileBytes = kLanes * 16;

template <int NA, int NB, int NC, int NW, bool NT, bool NTS>
__global__ __launch_bounds__(kLanes) void stream_probe_kernel(const char* __restrict__ a, const char* __restrict__ b,
                                                              const char* __restrict__ c, char* __restrict__ w,
                                                              int64_t row_bytes, uint32_t tiles_per_token,
                                                              unsigned* __restrict__ sink) {
  constexpr int NR = NA + NB + NC;
  extern __shared__ char occupancy_reserve[];
  (void)occupancy_reserve;
  const int64_t tok = blockIdx.x / tiles_per_token;
  const uint32_t col = (blockIdx.x % tiles_per_token) * kTileBytes + threadIdx.x * 16;
  // one span per array covering this token's rows
  const Span<char, true> sa(a + tok * NA * row_bytes, NA * row_bytes);
  const Span<char, true> sb(b + tok * NB * row_bytes, NB * row_bytes);
  const Span<char, true> sc(c + tok * NC * row_bytes, NC * row_bytes);
  const Span<char, true> sw(w + tok * NW * row_bytes, NW * row_bytes);
  u32x4 v[NR > 0 ? NR : 1];
#pragma unroll
  for (int i = 0; i < NA; ++i) v[i] = sa.load16<NT>((uint32_t)(i * row_bytes) + col);
#pragma unroll
  for (int i = 0; i < NB; ++i) v[NA + i] = sb.load16<NT>((uint32_t)(i * row_bytes) + col);
#pragma unroll
  for (int i = 0; i < NC; ++i) v[NA + NB + i] = sc.load16<NT>((uint32_t)(i * row_bytes) + col);
  __builtin_amdgcn_sched_barrier(0);
  // every input row feeds every output row, so no load can be dropped
  u32x4 tot = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < NR; ++i) tot += v[i];
  if constexpr (NW > 0) {
#pragma unroll
    for (int o = 0; o < NW; ++o) {
      u32x4 s = tot + u32x4{(uint32_t)o, 0u, 0u, 0u};
      if constexpr (NR > 0) s += v[o % NR];
      sw.store16<NTS>((uint32_t)(o * row_bytes) + col, s);
    }
  } else {
    if (tot.x == 0x9e3779b9u && tot.y == 0x7f4a7c15u && tot.z == tot.w) sink[threadIdx.x] = tot.x;
  }
}

// The same mixes for rows that are not a whole number of 4 KiB tiles (the
// layer kernels' flattened items): item i of the [T, row_bytes / 16] vector
// plane is token i / nvec, vector i % nvec, and a workgroup takes 256
// consecutive items, so it may span two tokens.
template <int NA, int NB, int NC, int NW, bool NT, bool NTS>
__global__ __launch_bounds__(kLanes) void stream_probe_flat_kernel(const char* __restrict__ a,
                                                                   const char* __restrict__ b,
                                                                   const char* __restrict__ c, char* __restrict__ w,
                                                                   int64_t row_bytes, int64_t tokens,
                                                                   unsigned* __restrict__ sink) {
  constexpr int NR = NA + NB + NC;
  extern __shared__ char occupancy_reserve[];
  (void)occupancy_reserve;
  const int64_t nvec = row_bytes / 16;
  const int64_t i0 = (int64_t)blockIdx.x * kLanes;
  const int64_t i = i0 + threadIdx.x;
  const int64_t t0 = i0 / nvec;
  int64_t t1 = (i0 + kLanes - 1) / nvec;
  if (t1 >= tokens) t1 = tokens - 1;
  const int64_t ntok = t1 - t0 + 1;
  const bool live = i < tokens * nvec;
  const int64_t tok = i / nvec;
  const uint32_t col = (uint32_t)((i - tok * nvec) * 16);
  const uint32_t trel = (uint32_t)(tok - t0);
  const Span<char, true> sa(a + t0 * NA * row_bytes, ntok * NA * row_bytes);
  const Span<char, true> sb(b + t0 * NB * row_bytes, ntok * NB * row_bytes);
  const Span<char, true> sc(c + t0 * NC * row_bytes, ntok * NC * row_bytes);
  const Span<char, true> sw(w + t0 * NW * row_bytes, ntok * NW * row_bytes);
  u32x4 v[NR > 0 ? NR : 1];
#pragma unroll
  for (int r = 0; r < NA; ++r) v[r] = live ? sa.load16<NT>((uint32_t)((trel * NA + r) * row_bytes) + col) : u32x4{};
#pragma unroll
  for (int r = 0; r < NB; ++r) v[NA + r] = live ? sb.load16<NT>((uint32_t)((trel * NB + r) * row_bytes) + col) : u32x4{};
#pragma unroll
  for (int r = 0; r < NC; ++r)
    v[NA + NB + r] = live ? sc.load16<NT>((uint32_t)((trel * NC + r) * row_bytes) + col) : u32x4{};
  __builtin_amdgcn_sched_barrier(0);
  u32x4 tot = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
  for (int r = 0; r < NR; ++r) tot += v[r];
  if constexpr (NW > 0) {
    if (live) {
#pragma unroll
      for (int o = 0; o < NW; ++o) {
        u32x4 s = tot + u32x4{(uint32_t)o, 0u, 0u, 0u};
        if constexpr (NR > 0) s += v[o % NR];
        sw.store16<NTS>((uint32_t)((trel * NW + o) * row_bytes) + col, s);
      }
    }
  } else {
    if (tot.x == 0x9e3779b9u && tot.y == 0x7f4a7c15u && tot.z == tot.w) sink[threadIdx.x] = tot.x;
  }
}

template <int NA, int NB, int NC, int NW, bool NT, bool NTS>
hipError_t launch_policy(const void* a, const void* b, const void* c, void* w, int64_t tokens, int64_t row_bytes,
                         size_t lds, unsigned* sink, hipStream_t st) {
  if (row_bytes % kTileBytes != 0) {
    const dim3 grid((unsigned)((tokens * (row_bytes / 16) + kLanes - 1) / kLanes));
    stream_probe_flat_kernel<NA, NB, NC, NW, NT, NTS><<<grid, kLanes, lds, st>>>(
        (const char*)a, (const char*)b, (const char*)c, (char*)w, row_bytes, tokens, sink);
    return hipGetLastError();
  }
  const uint32_t tpt = (uint32_t)(row_bytes / kTileBytes);
  const dim3 grid((unsigned)(tokens * tpt));
  stream_probe_kernel<NA, NB, NC, NW, NT, NTS><<<grid, kLanes, lds, st>>>(
      (const char*)a, (const char*)b, (const char*)c, (char*)w, row_bytes, tpt, sink);
  return hipGetLastError();
}

// policy: 0 plain loads and stores, 1 nt loads and stores, 2 nt loads and plain
// stores, 3 plain loads and nt stores
template <int NA, int NB, int NC, int NW>
hipError_t launch(const void* a, const void* b, const void* c, void* w, int64_t tokens, int64_t row_bytes,
                  size_t lds, int policy, unsigned* sink, hipStream_t st) {
  switch (policy) {
    case 0: return launch_policy<NA, NB, NC, NW, false, false>(a, b, c, w, tokens, row_bytes, lds, sink, st);
    case 1: return launch_policy<NA, NB, NC, NW, true, true>(a, b, c, w, tokens, row_bytes, lds, sink, st);
    case 2: return launch_policy<NA, NB, NC, NW, true, false>(a, b, c, w, tokens, row_bytes, lds, sink, st);
    default: return launch_policy<NA, NB, NC, NW, false, true>(a, b, c, w, tokens, row_bytes, lds, sink, st);
  }
}

}  // namespace

// Moves tokens x (na + nb + nc) input rows and tokens x nw output rows of
// row_bytes each (a multiple of 16; whole 4 KiB tiles per token when it is a
// multiple of 4096, flattened items otherwise).  Supported (na, nb, nc, nw): the read /
// write mixes of the layer's streaming kernels and the plain references
// (4,0,0,0) (4,0,0,1) (4,1,0,4) (4,1,0,1) (4,4,1,0) (1,0,0,1) (1,0,0,0)
// (0,0,0,1), and those of the standalone ops (4,0,0,5) (1,0,0,4) (4,4,1,4).  wg_per_cu > 0 caps resident workgroups per CU (0: no cap).
// nt is the cache policy: 0 plain, 1 nt (streaming) loads and stores, 2 nt
// loads with plain stores, 3 plain loads with nt stores.
// `sink` is 1 KiB of device memory that a read-only mix keeps live.  Returns
// 0, 1 for an unsupported mix, shape or a missing array, 2 for a launch error.
extern "C" int mhc_probe_stream(int na, int nb, int nc, int nw, const void* a, const void* b, const void* c, void* w,
                                int64_t tokens, int64_t row_bytes, int wg_per_cu, int nt, void* sink,
                                void* stream) {
  if (tokens <= 0 || row_bytes <= 0 || row_bytes % 16 != 0 || nt < 0 || nt > 3) return 1;
  if ((na > 0 && !a) || (nb > 0 && !b) || (nc > 0 && !c) || (nw > 0 && !w) || (nw == 0 && !sink)) return 1;
  int rows = na > nb ? na : nb;
  rows = rows > nc ? rows : nc;
  rows = rows > nw ? rows : nw;
  if ((int64_t)rows * row_bytes >= ((int64_t)1 << 31)) return 1;  // one token's span of an array
  if (tokens * (row_bytes / 16) / kLanes >= ((int64_t)1 << 31)) return 1;  // grid size
  const size_t lds = mhc::occupancy_lds(wg_per_cu);
  hipStream_t st = (hipStream_t)stream;
  unsigned* s = (unsigned*)sink;
  const int key = na * 1000 + nb * 100 + nc * 10 + nw;
  hipError_t e;
  switch (key) {
    case 4000: e = launch<4, 0, 0, 0>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4001: e = launch<4, 0, 0, 1>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4104: e = launch<4, 1, 0, 4>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4101: e = launch<4, 1, 0, 1>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4410: e = launch<4, 4, 1, 0>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 1001: e = launch<1, 0, 0, 1>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 1000: e = launch<1, 0, 0, 0>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 1: e = launch<0, 0, 0, 1>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4005: e = launch<4, 0, 0, 5>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 1004: e = launch<1, 0, 0, 4>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    case 4414: e = launch<4, 4, 1, 4>(a, b, c, w, tokens, row_bytes, lds, nt, s, st); break;
    default: return 1;
  }
  return e == hipSuccess ? 0 : 2;
}
