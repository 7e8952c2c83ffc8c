// The cost of a dependent kernel launch: a chain of launches of a kernel that
// does almost nothing (the first lane of each workgroup adds one to that
// workgroup's own counter), each launch ordered after the previous one on the
// stream, submitted as plain launches or as one captured graph.  The
// reference measures the same quantity for its frame plan: ~0.5 ms of GPU-side
// launch cost per frame outside a CUDA graph, ~1.6 us per launch inside one
// (README.md:20-26, 73; NOTES.md:48-50).
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

__global__ __launch_bounds__(64) void chain_tick_kernel(unsigned* __restrict__ c) {
  if (threadIdx.x == 0) c[blockIdx.x] += 1u;
}

}  // namespace

float time_launch_chain(int n, int workgroups, int mode, int reps, hipStream_t s) {
  CK_REQUIRE(n > 0 && n <= 100000 && workgroups > 0 && workgroups <= 65536 && reps > 0 && (mode == 0 || mode == 1),
             "launch_chain: 0 < n <= 100000, 0 < workgroups <= 65536, reps > 0, mode 0 (plain) or 1 (graph)");
  unsigned* c = nullptr;
  hipStream_t own = nullptr;   // the null stream cannot be captured: a stream of our own then
  hipEvent_t e0 = nullptr, e1 = nullptr;
  hipGraph_t g = nullptr;
  hipGraphExec_t ge = nullptr;
  float ms = 0.f;
  auto cleanup = [&]() {
    if (ge) (void)hipGraphExecDestroy(ge);
    if (g) (void)hipGraphDestroy(g);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (c) (void)hipFree(c);
    if (own) (void)hipStreamDestroy(own);
  };
  try {
    if (!s) {
      CK_HIP(hipStreamCreateWithFlags(&own, hipStreamNonBlocking));
      s = own;
    }
    CK_HIP(hipMalloc(&c, sizeof(unsigned) * workgroups));
    CK_HIP(hipMemsetAsync(c, 0, sizeof(unsigned) * workgroups, s));
    CK_HIP(hipEventCreate(&e0));
    CK_HIP(hipEventCreate(&e1));
    auto chain = [&]() {
      for (int i = 0; i < n; ++i) CK_LAUNCH(chain_tick_kernel, dim3(workgroups), dim3(64), 0, s, c);
    };
    if (mode == 1) {
      CK_HIP(hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
      try {
        chain();
      } catch (...) {
        hipGraph_t tmp = nullptr;
        (void)hipStreamEndCapture(s, &tmp);
        if (tmp) (void)hipGraphDestroy(tmp);
        throw;
      }
      CK_HIP(hipStreamEndCapture(s, &g));
      CK_HIP(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
      CK_HIP(hipGraphLaunch(ge, s));   // untimed first replay
    } else {
      chain();
    }
    CK_HIP(hipStreamSynchronize(s));
    CK_HIP(hipEventRecord(e0, s));
    for (int r = 0; r < reps; ++r) {
      if (mode == 1) CK_HIP(hipGraphLaunch(ge, s));
      else chain();
    }
    CK_HIP(hipEventRecord(e1, s));
    CK_HIP(hipEventSynchronize(e1));
    CK_HIP(hipEventElapsedTime(&ms, e0, e1));
  } catch (...) {
    if (s) (void)hipStreamSynchronize(s);
    cleanup();
    throw;
  }
  cleanup();
  return ms * 1e3f / ((float)n * reps);
}

}  // namespace ck
