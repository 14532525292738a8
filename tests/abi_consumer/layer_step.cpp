// A C++ consumer of the C ABI (include/mhc_abi.h) with no torch in the process:
// one dynamic HyperConnection layer step (forward, the closure, the closure's
// backward and the layer backward) through libmhc_hip.so on a stream of its
// own, plus the allocation-free forward, whose outputs must equal the
// workspace forward's bit for bit.  tests/test_gpu_abi_consumer.py writes the
// inputs, runs this program as a child process and checks the outputs against
// the float64 oracle.
//
//   layer_step <in.bin> <out.bin>
//
// in.bin:  int64 dtype, B, S, D, iters; float64 eps; then the raw arrays
//          H [B,S,4,D] (dtype), phi [4D,24] f32, H_pre_base [4], H_post_base [4],
//          H_res_base [16], alpha_pre, alpha_post, alpha_res [1 each] f32,
//          branch_output [B,S,D], dH_new [B,S,4,D], d_branch_input [B,S,D] (dtype).
// out.bin: branch_input, H_new, d_branch_output, dH (dtype); dH_post [B,4],
//          grad_phi [4D,24], grad_bias [24], grad_alpha [3], w [B,24], x [B,4D]
//          (f32); int64 1 if the allocation-free forward matched, else 0.
// Exit status 0 on success; otherwise the failing call and mhc_last_error().
#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/mhc_abi.h"

namespace {

#define HIP_OK(call)                                                              \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s: %s\n", #call, hipGetErrorString(e_));             \
      std::exit(2);                                                               \
    }                                                                             \
  } while (0)

#define MHC_OK_(call)                                                             \
  do {                                                                            \
    int rc_ = (call);                                                             \
    if (rc_ != MHC_OK) {                                                          \
      std::fprintf(stderr, "%s returned %d: %s\n", #call, rc_, mhc_last_error()); \
      std::exit(3);                                                               \
    }                                                                             \
  } while (0)

struct Reader {
  std::FILE* f;
  template <typename T>
  T scalar() {
    T v;
    if (std::fread(&v, sizeof(T), 1, f) != 1) { std::fprintf(stderr, "short input\n"); std::exit(4); }
    return v;
  }
  std::vector<char> bytes(size_t n) {
    std::vector<char> v(n);
    if (n && std::fread(v.data(), 1, n, f) != n) { std::fprintf(stderr, "short input\n"); std::exit(4); }
    return v;
  }
};

// A device copy of host bytes.
void* upload(const std::vector<char>& h) {
  void* d = nullptr;
  HIP_OK(hipMalloc(&d, h.size() ? h.size() : 1));
  if (!h.empty()) HIP_OK(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice));
  return d;
}

void* alloc(size_t n) {
  void* d = nullptr;
  HIP_OK(hipMalloc(&d, n ? n : 1));
  return d;
}

std::vector<char> download(const void* d, size_t n) {
  std::vector<char> h(n);
  if (n) HIP_OK(hipMemcpy(h.data(), d, n, hipMemcpyDeviceToHost));
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 3) {
    std::fprintf(stderr, "usage: %s <in.bin> <out.bin>\n", argv[0]);
    return 1;
  }
  std::FILE* fi = std::fopen(argv[1], "rb");
  if (!fi) { std::perror(argv[1]); return 1; }
  Reader rd{fi};
  const int dtype = (int)rd.scalar<int64_t>();
  const int64_t B = rd.scalar<int64_t>(), S = rd.scalar<int64_t>(), D = rd.scalar<int64_t>();
  const int iters = (int)rd.scalar<int64_t>();
  const float eps = (float)rd.scalar<double>();
  const size_t e = dtype == MHC_DTYPE_F32 ? 4 : 2;
  const size_t nH = (size_t)(B * S * 4 * D), nR = (size_t)(B * S * D), K = (size_t)(4 * D);
  void* H = upload(rd.bytes(nH * e));
  float* phi = (float*)upload(rd.bytes(K * 24 * 4));
  float* pre_base = (float*)upload(rd.bytes(16));
  float* post_base = (float*)upload(rd.bytes(16));
  float* res_base = (float*)upload(rd.bytes(64));
  float* a_pre = (float*)upload(rd.bytes(4));
  float* a_post = (float*)upload(rd.bytes(4));
  float* a_res = (float*)upload(rd.bytes(4));
  void* bo = upload(rd.bytes(nR * e));
  void* dHn = upload(rd.bytes(nH * e));
  void* dbi = upload(rd.bytes(nR * e));
  std::fclose(fi);

  hipStream_t st;
  HIP_OK(hipStreamCreate(&st));
  const size_t ws_bytes = mhc_layer_workspace_bytes(B, S, D, dtype);
  void* ws = alloc(ws_bytes);
  void* bi = alloc(nR * e);
  float* x = (float*)alloc(B * K * 4);
  float* w = (float*)alloc(B * 24 * 4);
  float* aux = (float*)alloc(B * 25 * 4);
  void* Hn = alloc(nH * e);
  void* dbo = alloc(nR * e);
  float* dpost = (float*)alloc(B * 4 * 4);
  void* dH = alloc(nH * e);
  float* gphi = (float*)alloc(K * 24 * 4);
  float* gbias = (float*)alloc(24 * 4);
  float* galpha = (float*)alloc(3 * 4);

  // forward, the closure, the closure's backward, the layer backward
  MHC_OK_(mhc_layer_dynamic_forward(H, dtype, phi, pre_base, post_base, res_base, a_pre, a_post, a_res, bi, x, w,
                                    aux, B, S, D, iters, eps, ws, ws_bytes, st));
  MHC_OK_(mhc_layer_add_forward(H, dtype, bo, dtype, w, Hn, B, S, D, st));
  MHC_OK_(mhc_layer_add_backward(dHn, dtype, bo, dtype, w, dbo, dpost, B, S, D, ws, ws_bytes, st));
  MHC_OK_(mhc_layer_dynamic_backward(H, dtype, dbi, dHn, dpost, phi, pre_base, post_base, res_base, a_pre, a_post,
                                     a_res, x, w, aux, dH, gphi, gbias, galpha, B, S, D, iters, eps, ws, ws_bytes,
                                     st));
  HIP_OK(hipStreamSynchronize(st));

  // the allocation-free forward into separate outputs, compared bit for bit
  void* bi2 = alloc(nR * e);
  float* x2 = (float*)alloc(B * K * 4);
  float* w2 = (float*)alloc(B * 24 * 4);
  float* aux2 = (float*)alloc(B * 25 * 4);
  MHC_OK_(mhc_layer_dynamic_forward_noalloc(H, dtype, phi, pre_base, post_base, res_base, a_pre, a_post, a_res, bi2,
                                            x2, w2, aux2, B, S, D, iters, eps, st));
  HIP_OK(hipStreamSynchronize(st));
  const bool same = download(bi, nR * e) == download(bi2, nR * e) && download(x, B * K * 4) == download(x2, B * K * 4) &&
                    download(w, B * 24 * 4) == download(w2, B * 24 * 4) &&
                    download(aux, B * 25 * 4) == download(aux2, B * 25 * 4);

  std::FILE* fo = std::fopen(argv[2], "wb");
  if (!fo) { std::perror(argv[2]); return 1; }
  auto put = [&](const void* d, size_t n) {
    const std::vector<char> h = download(d, n);
    if (n && std::fwrite(h.data(), 1, n, fo) != n) { std::fprintf(stderr, "short write\n"); std::exit(5); }
  };
  put(bi, nR * e);
  put(Hn, nH * e);
  put(dbo, nR * e);
  put(dH, nH * e);
  put(dpost, B * 4 * 4);
  put(gphi, K * 24 * 4);
  put(gbias, 24 * 4);
  put(galpha, 3 * 4);
  put(w, B * 24 * 4);
  put(x, B * K * 4);
  const int64_t flag = same ? 1 : 0;
  std::fwrite(&flag, sizeof flag, 1, fo);
  std::fclose(fo);

  for (void* p : {H, (void*)phi, (void*)pre_base, (void*)post_base, (void*)res_base, (void*)a_pre, (void*)a_post,
                  (void*)a_res, bo, dHn, dbi, ws, bi, (void*)x, (void*)w, (void*)aux, Hn, dbo, (void*)dpost, dH,
                  (void*)gphi, (void*)gbias, (void*)galpha, bi2, (void*)x2, (void*)w2, (void*)aux2})
    HIP_OK(hipFree(p));
  HIP_OK(hipStreamDestroy(st));
  std::printf("layer_step: B=%lld S=%lld D=%lld dtype=%d noalloc %s\n", (long long)B, (long long)S, (long long)D,
              dtype, same ? "same" : "DIFFERENT");
  return 0;
}
