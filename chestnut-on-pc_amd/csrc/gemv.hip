// Weight-streaming GEMV: the gfx950 replacement of the serial reduce
// `r_32_32_3_12288_32` (run_pinned2.py:989-1066; alu_opt.py:1-117).
//
// The reference runs a 12288-trip loop on one warp per block and later
// splits it over W warps with a shared-memory partial combine.  Here the
// reduction axis is spread over a whole 256-lane workgroup from the start:
//   * lane t of the workgroup owns columns step*2048 + 8t .. 8t+7 for every
//     2048-column step, and keeps its slice of x in registers for all rows;
//   * every W read is one 16-byte load per lane, fully coalesced (a wave
//     reads 1 KiB contiguous per instruction); RB rows are loaded before any
//     arithmetic so each lane has RB*NSTEP loads in flight.  W is read once
//     per frame and never again, so the loads are non-temporal (they do not
//     displace x and the activations from the caches), which measures
//     ~6% faster on the config-2 shape;
//   * workgroups are small (one 4-row batch each for up to 4096 rows): three
//     or more resident per CU keep more requests in flight than a few long
//     workgroups would (3072 rows: 768 workgroups);
//   * each lane accumulates its 8*NSTEP products in f32 (fixed order), the
//     wave sums its lanes with DPP row exchanges + readlane, and the four
//     wave partials are combined through LDS in wave order.
// The result is deterministic; relative to the exact sum it carries f32
// reassociation error only.
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_STEP_COLS = GEMV_THREADS * 8;   // 2048 columns per step
constexpr int GEMV_RB = 4;                          // rows per batch

template <int NSTEP>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(const half_t* __restrict__ W, const float* __restrict__ x,
                                                            const float* __restrict__ bias, float* __restrict__ y,
                                                            int rows, int K, int ldw, int rows_per_wg, int act) {
  __shared__ float red[2][4][GEMV_RB];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;

  float xr[NSTEP][8];
  bool cv[NSTEP];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int c = s * GEMV_STEP_COLS + t * 8;
    cv[s] = c < K;
    if (cv[s]) {
      float4_t a = *reinterpret_cast<const float4_t*>(x + c);
      float4_t b = *reinterpret_cast<const float4_t*>(x + c + 4);
      xr[s][0] = a[0]; xr[s][1] = a[1]; xr[s][2] = a[2]; xr[s][3] = a[3];
      xr[s][4] = b[0]; xr[s][5] = b[1]; xr[s][6] = b[2]; xr[s][7] = b[3];
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xr[s][j] = 0.f;
    }
  }

  const int r0 = blockIdx.x * rows_per_wg;
  const int r1 = min(rows, r0 + rows_per_wg);
  int par = 0;
  for (int rb = r0; rb < r1; rb += GEMV_RB, par ^= 1) {
    half8_t w[GEMV_RB][NSTEP];
#pragma unroll
    for (int i = 0; i < GEMV_RB; ++i) {
      const int r = min(rb + i, r1 - 1);   // tail rows re-read the last row; their sums are dropped
      const half_t* wr = W + (long)r * ldw + t * 8;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
        if (cv[s]) w[i][s] = __builtin_nontemporal_load(reinterpret_cast<const half8_t*>(wr + s * GEMV_STEP_COLS));
        else w[i][s] = half8_t{};
      }
    }
    float acc[GEMV_RB];
#pragma unroll
    for (int i = 0; i < GEMV_RB; ++i) {
      float a = 0.f;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) a = fmaf((float)w[i][s][j], xr[s][j], a);
      acc[i] = wave_sum(a);
    }
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < GEMV_RB; ++i) red[par][wave][i] = acc[i];
    }
    __syncthreads();
    if (t < GEMV_RB && rb + t < r1) {
      float v = ((red[par][0][t] + red[par][1][t]) + red[par][2][t]) + red[par][3][t];
      if (bias) v += bias[rb + t];
      if (act == GEMV_GELU) v = gelu_tanh(v);
      y[rb + t] = v;
    }
    // `red` is double-buffered by batch parity: the slot written two batches
    // later is only reused after every thread passed the next barrier.
  }
}

template <int NSTEP>
void launch_gemv_n(const half_t* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
                   int rpw, hipStream_t s) {
  const int grid = ceil_div(rows, rpw);
  hipLaunchKernelGGL(gemv_kernel<NSTEP>, dim3(grid), dim3(GEMV_THREADS), 0, s, W, x, bias, y, rows, K, ldw, rpw, act);
  CK_LAUNCHED("gemv");
}

}  // namespace

void launch_gemv(const half_t* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
                 int rows_per_wg, hipStream_t s) {
  CK_REQUIRE(W && x && y, "gemv: null pointer");
  CK_REQUIRE(rows > 0 && K > 0, "gemv: rows and K must be positive");
  CK_REQUIRE(K % 8 == 0, "gemv: K must be a multiple of 8");
  CK_REQUIRE(ldw >= K && ldw % 8 == 0, "gemv: ldw must be >= K and a multiple of 8");
  CK_REQUIRE(K <= 8 * GEMV_STEP_COLS, "gemv: K above 16384 is not supported");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(W) & 15) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0,
             "gemv: W and x must be 16-byte aligned");
  CK_REQUIRE(act == GEMV_NONE || act == GEMV_GELU, "gemv: unknown activation");
  int rpw = rows_per_wg;
  if (rpw <= 0) rpw = (rows + 1023) / 1024;         // >= 3 workgroups per CU up to 3072 rows
  rpw = ((rpw + GEMV_RB - 1) / GEMV_RB) * GEMV_RB;  // whole batches
  const int nstep = ceil_div(K, GEMV_STEP_COLS);
  switch (nstep) {
    case 1: launch_gemv_n<1>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 2: launch_gemv_n<2>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 3: launch_gemv_n<3>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 4: launch_gemv_n<4>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 5: launch_gemv_n<5>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 6: launch_gemv_n<6>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    case 7: launch_gemv_n<7>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
    default: launch_gemv_n<8>(W, x, bias, y, rows, K, ldw, act, rpw, s); break;
  }
}

}  // namespace ck
