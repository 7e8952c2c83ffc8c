// The operand stream of a block GEMM without its arithmetic: the grid, tile
// order, loads and waits of the 128x128 LDS-DMA tile (64-wide K-steps, A and
// B K-contiguous), with no MFMA, no fragment reads and no epilogue.  Its time
// against the GEMM's own says how much of the GEMM is the memory system
// delivering operands to the CUs.
//   mode 0: LDS-DMA (global_load_lds_dwordx4) into a 4-stage ring, 3 K-steps
//           ahead, 4 waves; per step a wait for the step's loads and a barrier
//   mode 1: the same with 8 waves issuing half the loads each
//   mode 2: 16-byte loads into registers 3 K-steps ahead, 4 waves, no LDS
//   mode 3: mode 0 on 128x96 tiles (the QKV GEMM's tile; N % 96 == 0)
// Operands rotate over `copies` distinct copies, so with enough of them the
// weights come from HBM as in a frame.
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr int BK_STREAM = 64;
constexpr int SBM = 128, SBN = 128;

// chunk c of step s: row c / 8 of the stage (SBM A rows, then the B rows),
// 16-byte column c % 8
__device__ __forceinline__ const half_t* stream_src(const half_t* A, const half_t* B, int m0, int n0, int K, int c,
                                                    int s) {
  const int row = c >> 3, col = (c & 7) * 8, k0 = s * BK_STREAM;
  return row < SBM ? A + (long)(m0 + row) * K + k0 + col : B + (long)(n0 + row - SBM) * K + k0 + col;
}

__device__ __forceinline__ void stream_tile(int Mt, int Nt, int bn, int& m0, int& n0) {
  const int total = Mt * Nt;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);   // the GEMM's XCD grouping
  m0 = (L % Mt) * SBM;
  n0 = (L / Mt) * bn;
}

// wave w's NI 1-KB loads of step s into ring stage st
template <int NI>
__device__ __forceinline__ void stream_issue(const half_t* A, const half_t* B, int m0, int n0, int K, int s, half_t* st,
                                             int w, int lane) {
#pragma unroll
  for (int i = 0; i < NI; ++i) {
    const int c = (w * NI + i) * 64 + lane;
    __builtin_amdgcn_global_load_lds(stream_src(A, B, m0, n0, K, c, s), (lds_ptr_t)(st + (w * NI + i) * 512), 16, 0, 0);
  }
}

// BN: the B tile's rows (128, or 96 for the QKV tile)
template <int NW, int BN>
__global__ __launch_bounds__(64 * NW) void stream_dma_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                                                             int Mt, int Nt, int K, unsigned* __restrict__ sink) {
  constexpr int SST = (SBM + BN) * BK_STREAM;   // stage: halves
  constexpr int NI = (SBM + BN) / 8 / NW;       // 1-KB load instructions per wave per step
  static_assert(NI * 8 * NW == SBM + BN, "the stage must split into whole load instructions per wave");
  __shared__ __attribute__((aligned(1024))) half_t lds[4 * SST];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  int m0, n0;
  stream_tile(Mt, Nt, BN, m0, n0);
  const int nk = K / BK_STREAM;
  stream_issue<NI>(A, B, m0, n0, K, 0, lds, w, lane);
  stream_issue<NI>(A, B, m0, n0, K, min(1, nk - 1), lds + SST, w, lane);
  stream_issue<NI>(A, B, m0, n0, K, min(2, nk - 1), lds + 2 * SST, w, lane);
  for (int s = 0; s < nk; ++s) {
    wait_vm_lgkm0<2 * NI>();   // step s has landed; the next two steps' loads may be in flight
    lds_barrier();
    // past the end: the last step again, into a stage never read
    stream_issue<NI>(A, B, m0, n0, K, min(s + 3, nk - 1), lds + ((s + 3) & 3) * SST, w, lane);
  }
  wait_vm_lgkm0<0>();
  if (threadIdx.x == 0) sink[blockIdx.x] = lds[lane];
}

__global__ __launch_bounds__(256) void stream_vgpr_kernel(const half_t* __restrict__ A, const half_t* __restrict__ B,
                                                          int Mt, int Nt, int K, unsigned* __restrict__ sink) {
  const int t = threadIdx.x;
  int m0, n0;
  stream_tile(Mt, Nt, SBN, m0, n0);
  const int nk = K / BK_STREAM;
  u32x4_t r[3][8];
  u32x4_t x = {0u, 0u, 0u, 0u};
  auto ld = [&](u32x4_t (&q)[8], int s) {
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = *reinterpret_cast<const u32x4_t*>(stream_src(A, B, m0, n0, K, t + 256 * i, s));
  };
  ld(r[0], 0);
  ld(r[1], min(1, nk - 1));
  ld(r[2], min(2, nk - 1));
  for (int s = 0; s < nk; s += 3) {
#pragma unroll
    for (int b = 0; b < 3; ++b) {
      if (s + b < nk) {
        wait_vm_lgkm0<16>();   // the oldest buffer has landed
#pragma unroll
        for (int i = 0; i < 8; ++i) x ^= r[b][i];
        lds_barrier();
        ld(r[b], min(s + b + 3, nk - 1));
      }
    }
  }
  wait_vm_lgkm0<0>();
  if (t == 0) sink[blockIdx.x] = x[0] ^ x[1] ^ x[2] ^ x[3];
}

}  // namespace

float time_operand_stream(int M, int N, int K, int mode, int copies, int reps, hipStream_t s) {
  CK_REQUIRE(mode >= 0 && mode <= 3 && copies >= 1 && copies <= 64 && reps > 0,
             "operand_stream: mode 0-3, 1 <= copies <= 64, reps > 0");
  const int bn = mode == 3 ? 96 : SBN;
  CK_REQUIRE(M > 0 && N > 0 && K > 0 && M % SBM == 0 && N % bn == 0 && K % BK_STREAM == 0,
             "operand_stream: M a multiple of 128, N of the tile width (128; 96 in mode 3), K of 64");
  CK_REQUIRE((long)(M / SBM) * (N / bn) <= 65536, "operand_stream: at most 65536 tiles");
  const size_t na = (size_t)M * K, nb = (size_t)N * K;
  CK_REQUIRE((na + nb) * 2 * copies <= (size_t(32) << 30), "operand_stream: at most 32 GiB of operand copies");
  const int Mt = M / SBM, Nt = N / bn, grid = Mt * Nt;
  half_t* buf = nullptr;
  unsigned* sink = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
  float ms = 0.f;
  auto cleanup = [&]() {
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (buf) (void)hipFree(buf);
    if (sink) (void)hipFree(sink);
  };
  try {
    CK_HIP(hipMalloc(&buf, (na + nb) * 2 * copies));
    CK_HIP(hipMalloc(&sink, sizeof(unsigned) * grid));
    CK_HIP(hipMemsetAsync(buf, 0x3c, (na + nb) * 2 * copies, s));
    CK_HIP(hipEventCreate(&e0));
    CK_HIP(hipEventCreate(&e1));
    auto launch = [&](int i) {
      const half_t* A = buf + (size_t)(i % copies) * (na + nb);
      const half_t* B = A + na;
      if (mode == 0) CK_LAUNCH((stream_dma_kernel<4, 128>), dim3(grid), dim3(256), 0, s, A, B, Mt, Nt, K, sink);
      else if (mode == 1) CK_LAUNCH((stream_dma_kernel<8, 128>), dim3(grid), dim3(512), 0, s, A, B, Mt, Nt, K, sink);
      else if (mode == 3) CK_LAUNCH((stream_dma_kernel<4, 96>), dim3(grid), dim3(256), 0, s, A, B, Mt, Nt, K, sink);
      else CK_LAUNCH(stream_vgpr_kernel, dim3(grid), dim3(256), 0, s, A, B, Mt, Nt, K, sink);
    };
    for (int i = 0; i < reps; ++i) launch(i);   // untimed: clocks up, caches in their steady state
    CK_HIP(hipEventRecord(e0, s));
    for (int i = 0; i < reps; ++i) launch(i);
    CK_HIP(hipEventRecord(e1, s));
    CK_HIP(hipEventSynchronize(e1));
    CK_HIP(hipEventElapsedTime(&ms, e0, e1));
  } catch (...) {
    (void)hipStreamSynchronize(s);
    cleanup();
    throw;
  }
  cleanup();
  return ms * 1e3f / (float)reps;
}

}  // namespace ck
