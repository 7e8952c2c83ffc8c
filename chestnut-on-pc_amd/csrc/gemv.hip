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
//     arithmetic so each lane has RB*NSTEP loads in flight.  For weights that
//     stream (the config-2 shape, the 1B model's 2 GB) the loads are
//     non-temporal: they do not displace x and the activations from the
//     caches (config 2: 13.8 against 15.0 us).  A model whose weights fit the
//     256 MB Infinity Cache (the 39M model) loads them with the default policy
//     and finds them there the next frame (-1.1% of its frame); the caller
//     chooses (`stream`);
//   * workgroups are small (one 4-row batch each for up to 4096 rows): three
//     or more resident per CU keep more requests in flight than a few long
//     workgroups would (3072 rows: 768 workgroups);
//   * each lane accumulates its 8*NSTEP products in f32 (fixed order), the
//     wave sums its lanes with DPP row exchanges + readlane, and the four
//     wave partials are combined through LDS in wave order.
// The result is deterministic; relative to the exact sum it carries f32
// reassociation error only.
//
// A launch can carry two independent GEMVs (the GRU's input and hidden
// products: one launch instead of two), and the input vector can be the GRU
// update computed on the fly from the gate pre-activations (the heads GEMV
// after the GRU: the gate kernel is folded into it).
#include <algorithm>

#include "common.h"
#include "im2col_u8.h"
#include "kernels.h"

namespace ck {
namespace {

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
};

// Workgroup `bid` of a GEMV launch (the body of gemv_kernel, also run by the
// GEMV workgroups of gemv_im2col_kernel).
template <int NSTEP, bool GATE, bool NT>
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
        const float4_t u = *reinterpret_cast<const float4_t*>(a.x + c);
        const float4_t v = *reinterpret_cast<const float4_t*>(a.x + c + 4);
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

template <int NSTEP, bool GATE, bool NT>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(const GemvArgs a0, const GemvArgs a1, int nb0) {
  gemv_block<NSTEP, GATE, NT>(a0, a1, nb0, (int)blockIdx.x);
}

// Layer-1 im2col of the conv stem (im2col_u8_gather) for `batch` images,
// `blocks_per_image` 256-thread blocks each.  In the shared launch its
// blocks are folded onto `nblk` workgroups, U blocks per workgroup.
struct Im2colU8Args {
  const uint8_t* img;
  half_t* patches;
  int C, H, W, Kp, Ho, Wo, batch, blocks_per_image, nblk;
};

// One launch for two independent pieces of work that each leave part of the
// chip idle: workgroups [0, nb) run the GEMV `a`, the next `nblk` the
// im2col.  The GEMV's workgroups come first so its weight stream starts at
// once; the im2col's take the slots the GEMV leaves free (the host sizes
// nblk to them), each running U (1-4) of the im2col's blocks with every gather
// load issued before the first store, so the whole im2col is resident in one
// round beside the GEMV (the temporal GEMV and stem layer 1 both wait only on
// the policy inputs).
template <int NSTEP, bool NT, int U>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_im2col_kernel(const GemvArgs a, int nb, const Im2colU8Args c) {
  const int bid = (int)blockIdx.x;
  if (bid < nb) {
    gemv_block<NSTEP, false, NT>(a, a, nb, bid);
    return;
  }
  const int total = c.batch * c.blocks_per_image;
  half8_t v[U];
  long off[U];
  bool ok[U];
  const int per = c.Ho * c.Wo * (c.Kp / 8);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // clamped to the last valid block and item (their stores are dropped),
    // so no gather sits under a branch and all U gathers issue together
    const int j0 = bid - nb + u * c.nblk, j = min(j0, total - 1);
    const int b = j / c.blocks_per_image;
    const int i0 = (j - b * c.blocks_per_image) * GEMV_THREADS + (int)threadIdx.x, i = min(i0, per - 1);
    im2col_u8_gather(c.img, c.C, c.H, c.W, c.Kp, c.Ho, c.Wo, b, i, v[u], off[u]);
    ok[u] = j0 < total && i0 < per;
  }
  // device-scope stores: the layer-1 conv GEMM reads the patches next
  const auto rsrc = sc1_rsrc(c.patches, 2L * c.batch * c.Ho * c.Wo * c.Kp);
#pragma unroll
  for (int u = 0; u < U; ++u)
    if (ok[u]) store_sc1(rsrc, off[u], v[u]);
}

GemvArgs make_args(const half_t* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
                   int rows_per_wg) {
  GemvArgs a{};
  a.W = W; a.x = x; a.bias = bias; a.y = y;
  a.rows = rows; a.K = K; a.ldw = ldw; a.act = act; a.rows_per_wg = rows_per_wg;
  return a;
}

void check_args(const GemvArgs& a) {
  CK_REQUIRE(a.W && a.y && (a.x || a.gi), "gemv: null pointer");
  CK_REQUIRE(a.rows > 0 && a.K > 0, "gemv: rows and K must be positive");
  CK_REQUIRE(a.K % 8 == 0, "gemv: K must be a multiple of 8");
  CK_REQUIRE(a.ldw >= a.K && a.ldw % 8 == 0, "gemv: ldw must be >= K and a multiple of 8");
  CK_REQUIRE(a.K <= 8 * GEMV_STEP_COLS, "gemv: K above 16384 is not supported");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(a.W) & 15) == 0 && (reinterpret_cast<uintptr_t>(a.x) & 15) == 0,
             "gemv: W and x must be 16-byte aligned");
  CK_REQUIRE(!a.gi || (a.gh && a.hp && a.h1), "gemv: the GRU-gated input needs gi, gh, h_prev and an output for h");
  CK_REQUIRE(!a.gi || ((reinterpret_cast<uintptr_t>(a.gi) | reinterpret_cast<uintptr_t>(a.gh) |
                        reinterpret_cast<uintptr_t>(a.hp)) & 15) == 0,
             "gemv: gi, gh and h_prev must be 16-byte aligned");
  CK_REQUIRE(a.act == GEMV_NONE || a.act == GEMV_GELU, "gemv: unknown activation");
}

int batch_rows(const GemvArgs& a) {
  int rpw = a.rows_per_wg;
  if (rpw <= 0) rpw = (a.rows + 1023) / 1024;          // >= 3 workgroups per CU up to 3072 rows
  return ((rpw + GEMV_RB - 1) / GEMV_RB) * GEMV_RB;    // whole batches
}

template <int NSTEP, bool GATE>
void launch_n(GemvArgs a0, GemvArgs a1, bool two, bool nt, hipStream_t s) {
  a0.rows_per_wg = batch_rows(a0);
  const int nb0 = ceil_div(a0.rows, a0.rows_per_wg);
  int grid = nb0;
  if (two) {
    a1.rows_per_wg = batch_rows(a1);
    grid += ceil_div(a1.rows, a1.rows_per_wg);
  } else {
    a1 = a0;
  }
  if (nt) CK_LAUNCH((gemv_kernel<NSTEP, GATE, true>), dim3(grid), dim3(GEMV_THREADS), 0, s, a0, a1, nb0);
  else CK_LAUNCH((gemv_kernel<NSTEP, GATE, false>), dim3(grid), dim3(GEMV_THREADS), 0, s, a0, a1, nb0);
  CK_LAUNCHED("gemv");
}

template <bool GATE>
void launch_args(const GemvArgs& a0, const GemvArgs& a1, bool two, bool nt, hipStream_t s) {
  const int nstep = ceil_div(two ? std::max(a0.K, a1.K) : a0.K, GEMV_STEP_COLS);
  switch (nstep) {
    case 1: launch_n<1, GATE>(a0, a1, two, nt, s); break;
    case 2: launch_n<2, GATE>(a0, a1, two, nt, s); break;
    case 3: launch_n<3, GATE>(a0, a1, two, nt, s); break;
    case 4: launch_n<4, GATE>(a0, a1, two, nt, s); break;
    case 5: launch_n<5, GATE>(a0, a1, two, nt, s); break;
    case 6: launch_n<6, GATE>(a0, a1, two, nt, s); break;
    case 7: launch_n<7, GATE>(a0, a1, two, nt, s); break;
    default: launch_n<8, GATE>(a0, a1, two, nt, s); break;
  }
}

// Resident workgroups of the shared launch over the whole current device.
template <int NSTEP, bool NT>
int resident_slots() {
  int dev = 0, per_cu = 0, cus = 0;
  CK_HIP(hipGetDevice(&dev));
  CK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  CK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, reinterpret_cast<const void*>(gemv_im2col_kernel<NSTEP, NT, 1>), GEMV_THREADS, 0));
  return std::max(1, per_cu) * std::max(1, cus);
}

template <int NSTEP, bool NT, int U>
void launch_fused_u(const GemvArgs& a, int nb, const Im2colU8Args& c, hipStream_t s) {
  CK_LAUNCH((gemv_im2col_kernel<NSTEP, NT, U>), dim3((unsigned)(nb + c.nblk)), dim3(GEMV_THREADS), 0, s, a, nb, c);
}

template <int NSTEP, bool NT>
void launch_fused(GemvArgs a, Im2colU8Args c, int slots, hipStream_t s) {
  a.rows_per_wg = batch_rows(a);
  const int nb = ceil_div(a.rows, a.rows_per_wg);
  const long total = (long)c.batch * c.blocks_per_image;
  CK_REQUIRE(total < (1L << 30), "gemv_im2col_u8: image too large");
  // the slots the GEMV leaves free, at least a quarter of the im2col's blocks
  const long free_slots = std::max<long>((long)slots - nb, ceil_div(total, 4));
  const int U = (int)std::min<long>(4, ceil_div(total, free_slots));
  c.nblk = ceil_div(total, U);
  if (U == 1) launch_fused_u<NSTEP, NT, 1>(a, nb, c, s);
  else if (U == 2) launch_fused_u<NSTEP, NT, 2>(a, nb, c, s);
  else if (U == 3) launch_fused_u<NSTEP, NT, 3>(a, nb, c, s);
  else launch_fused_u<NSTEP, NT, 4>(a, nb, c, s);
  CK_LAUNCHED("gemv_im2col_u8");
}

template <int NSTEP>
void launch_fused_nt(const GemvArgs& a, const Im2colU8Args& c, bool nt, int slots, hipStream_t s) {
  if (slots <= 0) slots = nt ? resident_slots<NSTEP, true>() : resident_slots<NSTEP, false>();
  if (nt) launch_fused<NSTEP, true>(a, c, slots, s);
  else launch_fused<NSTEP, false>(a, c, slots, s);
}

template <int NSTEP>
int slots_nt(bool nt) {
  return nt ? resident_slots<NSTEP, true>() : resident_slots<NSTEP, false>();
}

}  // namespace

int gemv_workgroups(int rows) {
  CK_REQUIRE(rows > 0, "gemv: rows must be positive");
  GemvArgs a{};
  a.rows = rows;
  return ceil_div(rows, batch_rows(a));
}

int gemv_im2col_u8_slots(int K, bool stream) {
  CK_REQUIRE(K > 0 && K <= 8 * GEMV_STEP_COLS, "gemv_im2col_u8: K must be in (0, 16384]");
  switch (ceil_div(K, GEMV_STEP_COLS)) {
    case 1: return slots_nt<1>(stream);
    case 2: return slots_nt<2>(stream);
    case 3: return slots_nt<3>(stream);
    case 4: return slots_nt<4>(stream);
    case 5: return slots_nt<5>(stream);
    case 6: return slots_nt<6>(stream);
    case 7: return slots_nt<7>(stream);
    default: return slots_nt<8>(stream);
  }
}

void launch_gemv_im2col_u8(const half_t* Wt, const float* x, const float* bias, float* y, int rows, int K, int act,
                           bool stream, const uint8_t* img, int batch, int C, int H, int W, half_t* patches, int Kp,
                           int slots, hipStream_t s) {
  const GemvArgs a = make_args(Wt, x, bias, y, rows, K, K, act, 0);
  check_args(a);
  CK_REQUIRE(img && patches && batch > 0 && C > 0 && H > 0 && W > 0, "gemv_im2col_u8: bad im2col arguments");
  CK_REQUIRE(Kp >= 9 * C && Kp % 8 == 0, "gemv_im2col_u8: Kp must be >= 9C and a multiple of 8");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(patches) & 15) == 0, "gemv_im2col_u8: patches must be 16-byte aligned");
  Im2colU8Args c{};
  c.img = img; c.patches = patches; c.C = C; c.H = H; c.W = W; c.Kp = Kp; c.batch = batch;
  c.Ho = (H - 1) / 2 + 1;
  c.Wo = (W - 1) / 2 + 1;
  const long per = (long)c.Ho * c.Wo * (Kp / 8);
  CK_REQUIRE(per < (1L << 31) && (long)H * W < (1L << 31), "gemv_im2col_u8: image too large");
  c.blocks_per_image = (int)ceil_div(per, GEMV_THREADS);
  switch (ceil_div(K, GEMV_STEP_COLS)) {
    case 1: launch_fused_nt<1>(a, c, stream, slots, s); break;
    case 2: launch_fused_nt<2>(a, c, stream, slots, s); break;
    case 3: launch_fused_nt<3>(a, c, stream, slots, s); break;
    case 4: launch_fused_nt<4>(a, c, stream, slots, s); break;
    case 5: launch_fused_nt<5>(a, c, stream, slots, s); break;
    case 6: launch_fused_nt<6>(a, c, stream, slots, s); break;
    case 7: launch_fused_nt<7>(a, c, stream, slots, s); break;
    default: launch_fused_nt<8>(a, c, stream, slots, s); break;
  }
}

void launch_gemv(const half_t* W, const float* x, const float* bias, float* y, int rows, int K, int ldw, int act,
                 int rows_per_wg, hipStream_t s, bool stream) {
  const GemvArgs a = make_args(W, x, bias, y, rows, K, ldw, act, rows_per_wg);
  check_args(a);
  launch_args<false>(a, a, false, stream, s);
}

void launch_gemv2(const half_t* W0, const float* x0, const float* b0, float* y0, int rows0, int K0, const half_t* W1,
                  const float* x1, const float* b1, float* y1, int rows1, int K1, hipStream_t s, bool stream) {
  const GemvArgs a0 = make_args(W0, x0, b0, y0, rows0, K0, K0, GEMV_NONE, 0);
  const GemvArgs a1 = make_args(W1, x1, b1, y1, rows1, K1, K1, GEMV_NONE, 0);
  check_args(a0);
  check_args(a1);
  launch_args<false>(a0, a1, true, stream, s);
}

void launch_gemv_gru(const half_t* W, const float* bias, float* y, int rows, const float* gi, const float* gh,
                     const float* h_prev, float* h_out, float* h_out2, int H, hipStream_t s, bool stream) {
  GemvArgs a = make_args(W, nullptr, bias, y, rows, H, H, GEMV_NONE, 0);
  a.gi = gi; a.gh = gh; a.hp = h_prev; a.h1 = h_out; a.h2 = h_out2;
  check_args(a);
  launch_args<true>(a, a, false, stream, s);
}

}  // namespace ck
