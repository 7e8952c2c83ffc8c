// The weight-streaming GEMV's workgroup body (gemv.hip) as a device
// function, with its argument block.
#pragma once

#include "common.h"
#include "kernels.h"
#include "policy_inputs.h"

namespace ck {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_STEP_COLS = GEMV_THREADS * 8;   // 2048 columns per step
constexpr int GEMV_RB = 4;                          // rows per batch

// One GEMV of a launch.  Workgroups [0, nb0) take the first, the rest the
// second (when the launch carries two).
struct GemvArgs {
  const half_t* W;
  const float* x;      // input vector (null when GRU-gated)
  const float* bias;
  float* y;
  int rows, K, ldw, rows_per_wg, act;
  // GRU-gated input (gates r, z, n as rows [0,K), [K,2K), [2K,3K) of gi and
  // gh, biases included): r = sig(gi_r + gh_r), z = sig(gi_z + gh_z),
  // n = tanh(gi_n + r * gh_n), x = (1 - z) * n + z * hp.  The first
  // workgroup also stores x to h1 (and h2 when given).
  const float* gi;
  const float* gh;
  const float* hp;
  float* h1;
  float* h2;
  // Feature-ring input (gemv_block XR): x[k*xlen + c] is entry c of frame
  // f = n - (xfL - 1) + xfs*k of the feature ring (ring slot f mod xfL), or of
  // xprev when f = n, n the frame counter at xcounter -- the features buffer
  // of the policy inputs (policy_inputs.h), read where it lies.
  const float* xring;
  const float* xprev;
  const unsigned* xcounter;
  int xfs, xlen, xfL;
};

// Workgroup `bid` of a GEMV launch (the body of gemv_kernel, also run by the
// GEMV workgroups of gemv_im2col_kernel).
template <int NSTEP, bool GATE, bool NT, bool XR = false>
__device__ __forceinline__ void gemv_block(const GemvArgs& a0, const GemvArgs& a1, int nb0, int bid) {
  __shared__ float red[2][4][GEMV_RB];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool second = bid >= nb0;
  const GemvArgs& a = second ? a1 : a0;
  const int blk = second ? bid - nb0 : bid;
  const half_t* __restrict__ W = a.W;
  const int rows = a.rows, K = a.K, ldw = a.ldw;

  const int r0 = blk * a.rows_per_wg;
  const int r1 = min(rows, r0 + a.rows_per_wg);
  // W batch loads: RB rows x NSTEP 16-byte chunks per lane.  With the
  // GRU-gated input the first batch is issued before the gates are
  // evaluated, so its latency overlaps that work; the plain form loads each
  // batch at the top of its iteration (an early load there costs registers
  // and occupancy on the wide GEMVs).
  half8_t w[GEMV_RB][NSTEP];
  auto load_batch = [&](int rb) {
#pragma unroll
    for (int i = 0; i < GEMV_RB; ++i) {
      const int r = min(rb + i, r1 - 1);   // tail rows re-read the last row; their sums are dropped
      const half_t* wr = W + (long)r * ldw;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s) {
        const int c = s * GEMV_STEP_COLS + t * 8;
        if (GATE) {
          // columns past K re-read the row's last chunk (in bounds, finite)
          // and meet x = 0, adding exact zeros: without a branch the gate
          // loads and arithmetic need not wait for these loads
          const half8_t* p = reinterpret_cast<const half8_t*>(wr + min(c, K - 8));
          w[i][s] = NT ? __builtin_nontemporal_load(p) : *p;
        } else if (c < K) {
          // the branch keeps every load of the batch ahead of the first FMA
          // (branch-free, the compiler interleaves loads with the FMAs and
          // holds about 2 in flight per lane instead of RB*NSTEP)
          const half8_t* p = reinterpret_cast<const half8_t*>(wr + c);
          w[i][s] = NT ? __builtin_nontemporal_load(p) : *p;
        } else {
          w[i][s] = half8_t{};
        }
      }
    }
  };
  if (GATE && r0 < r1) load_batch(r0);

  float xr[NSTEP][8];
#pragma unroll
  for (int s = 0; s < NSTEP; ++s) {
    const int c = s * GEMV_STEP_COLS + t * 8;
    if (c < K) {
      if (GATE) {
        // all seven 8-float slices are loaded before any gate is evaluated
        const float* src[7] = {a.gi + c, a.gi + K + c, a.gi + 2 * K + c, a.gh + c, a.gh + K + c, a.gh + 2 * K + c,
                               a.hp + c};
        float4_t g[7][2];
#pragma unroll
        for (int q = 0; q < 7; ++q) {
          g[q][0] = *reinterpret_cast<const float4_t*>(src[q]);
          g[q][1] = *reinterpret_cast<const float4_t*>(src[q] + 4);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int h = j >> 2, e = j & 3;
          const float r = sigmoidf_(g[0][h][e] + g[3][h][e]);
          const float z = sigmoidf_(g[1][h][e] + g[4][h][e]);
          const float n = tanhf(g[2][h][e] + r * g[5][h][e]);
          xr[s][j] = (1.0f - z) * n + z * g[6][h][e];
        }
        if (blk == 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            a.h1[c + j] = xr[s][j];
            if (a.h2) a.h2[c + j] = xr[s][j];
          }
        }
      } else {
        const float* src = a.x + c;
        if (XR) {   // the 8 columns lie in one ring entry (xlen % 8 == 0)
          const long n = a.xcounter[0];
          const int k = c / a.xlen, off = c - k * a.xlen;
          const long f = n - (a.xfL - 1) + (long)a.xfs * k;
          src = (f == n) ? a.xprev + off : a.xring + (long)wrap(f, a.xfL) * a.xlen + off;
        }
        const float4_t u = *reinterpret_cast<const float4_t*>(src);
        const float4_t v = *reinterpret_cast<const float4_t*>(src + 4);
        xr[s][0] = u[0]; xr[s][1] = u[1]; xr[s][2] = u[2]; xr[s][3] = u[3];
        xr[s][4] = v[0]; xr[s][5] = v[1]; xr[s][6] = v[2]; xr[s][7] = v[3];
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) xr[s][j] = 0.f;
    }
  }

  int par = 0;
  for (int rb = r0; rb < r1; rb += GEMV_RB, par ^= 1) {
    if (!GATE || rb != r0) load_batch(rb);
    float part[GEMV_RB];
#pragma unroll
    for (int i = 0; i < GEMV_RB; ++i) {
      float v = 0.f;
#pragma unroll
      for (int s = 0; s < NSTEP; ++s)
#pragma unroll
        for (int j = 0; j < 8; ++j) v = fmaf((float)w[i][s][j], xr[s][j], v);
      part[i] = v;
    }
    float acc[GEMV_RB];
#pragma unroll
    for (int i = 0; i < GEMV_RB; ++i) acc[i] = wave_sum(part[i]);
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < GEMV_RB; ++i) red[par][wave][i] = acc[i];
    }
    __syncthreads();
    if (t < GEMV_RB && rb + t < r1) {
      float v = ((red[par][0][t] + red[par][1][t]) + red[par][2][t]) + red[par][3][t];
      if (a.bias) v += a.bias[rb + t];
      if (a.act == GEMV_GELU) v = gelu_tanh(v);
      a.y[rb + t] = v;
    }
    // `red` is double-buffered by batch parity: the slot written two batches
    // later is only reused after every thread passed the next barrier.
  }
}

// Rows per workgroup: `rpw` rounded up to whole 4-row batches, or for rpw <= 0
// the automatic choice, three or more workgroups per CU up to 3072 rows.
inline int gemv_rows_per_wg(int rows, int rpw) {
  if (rpw <= 0) rpw = (rows + 1023) / 1024;
  return ((rpw + GEMV_RB - 1) / GEMV_RB) * GEMV_RB;
}

}  // namespace ck
