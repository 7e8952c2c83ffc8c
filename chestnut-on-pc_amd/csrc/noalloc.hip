// ck_gemm_noalloc: the GEMM entry point for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It is ck_gemm without the workspace
// argument: the split-K partials (and, for the tiles that need it, the
// transposed [K][N] B) live in `scratch`, a file-scope device array of
// kScratchBytes that each GPU the library runs on holds until the process
// ends.  The kernels are ck_gemm's own and take the array's device address
// as their workspace pointer.
//
// Host code never names `scratch` outside HIP_SYMBOL: in host code the name
// is a host-side stand-in, not a device address.  The device address is
// looked up once per device with hipGetSymbolAddress (with that device
// current) on the first call made on it, and cached per device; each GPU
// holds its own copy of the array at its own address.
//
// Nothing in the scratch has to start at zero: every split-K partial plane
// and every transposed-B element a call reads was written earlier in the
// same call, in stream order.  Calls share their GPU's array, so two calls
// that overlap on one GPU (different streams, or host threads without
// ordering) race on it.
#include <mutex>

#include "../../include/chestnut.h"
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr size_t kScratchBytes = size_t(32) << 20;   // 32 MiB per device
constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

std::mutex g_scratch_mu;
float* g_scratch_dev[kMaxDevices] = {};

// Device address of this device's `scratch` (looked up on first use).
float* scratch_on_current_device() {
  int dev = -1;
  CK_HIP(hipGetDevice(&dev));
  CK_REQUIRE(dev >= 0 && dev < kMaxDevices, "ck_gemm_noalloc: device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    CK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    CK_REQUIRE(p != nullptr && (reinterpret_cast<uintptr_t>(p) & 255) == 0,
               "ck_gemm_noalloc: scratch symbol has no aligned device address");
    g_scratch_dev[dev] = static_cast<float*>(p);
  }
  return g_scratch_dev[dev];
}

}  // namespace
}  // namespace ck

extern "C" int ck_gemm_noalloc(const void* A, const void* B, float* C, const float* bias, int M, int N, int K,
                               long lda, long ldb, long ldc, int b_kn, int tile, int split_k, void* stream) {
  try {
    ck::GemmDesc d;
    d.A = static_cast<const ck::half_t*>(A);
    d.B = static_cast<const ck::half_t*>(B);
    d.C = C;
    d.bias = bias;
    d.M = M; d.N = N; d.K = K;
    d.lda = lda; d.ldb = ldb; d.ldc = ldc;
    d.b_kn = b_kn != 0;
    d.epi = ck::EPI_F32;
    d.tile = tile;
    d.split = split_k;
    ck::GemmDesc plan = d;
    const size_t need = ck::gemm_plan(plan) * sizeof(float);
    CK_REQUIRE(need <= ck::kScratchBytes,
               "ck_gemm_noalloc: this GEMM needs " + std::to_string(need) + " bytes of workspace (split " +
                   std::to_string(plan.split) + "), above the " + std::to_string(ck::kScratchBytes) +
                   "-byte static scratch; use a smaller split_k or ck_gemm with a workspace");
    if (need) {
      // the cached address is the current device's copy of the array; the
      // kernels run on the stream's device, so the two must be the same GPU
      if (stream) {
        hipDevice_t sdev = -1;
        int cur = -1;
        CK_HIP(hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev));
        CK_HIP(hipGetDevice(&cur));
        CK_REQUIRE(sdev == cur, "ck_gemm_noalloc: the stream belongs to device " + std::to_string(sdev) +
                                    ", not the current device " + std::to_string(cur));
      }
      d.ws = ck::scratch_on_current_device();
      d.ws_floats = ck::kScratchBytes / sizeof(float);
    }
    ck::launch_gemm(d, static_cast<hipStream_t>(stream));
  } catch (const std::exception& ex) {
    ck::set_last_error(ex.what());
    return 1;
  } catch (...) {
    ck::set_last_error("unknown native exception");
    return 1;
  }
  return 0;
}
