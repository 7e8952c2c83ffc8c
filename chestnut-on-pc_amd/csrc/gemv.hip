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
// after the GRU: the gate kernel is folded into it).  The workgroup body
// (gemv_block.h) also runs inside other launches: the frame head below (the
// temporal GEMV beside the policy inputs and stem layer 1's im2col) and the
// split-K reduce of gemm.hip (the context GEMV).
#include <algorithm>

#include "common.h"
#include "gemv_block.h"
#include "im2col_u8.h"
#include "kernels.h"
#include "policy_inputs.h"

namespace ck {
namespace {

template <int NSTEP, bool GATE, bool NT>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(const GemvArgs a0, const GemvArgs a1, int nb0) {
  gemv_block<NSTEP, GATE, NT>(a0, a1, nb0, (int)blockIdx.x);
}

// K <= 512: one wave spans a row (lane l: columns 8l..8l+7), so the four
// waves of a workgroup take rows of their own, RW each, all loaded at once,
// and a row's sum is the wave sum alone: no LDS combine and no barrier (the
// workgroup form leaves three of its four waves without columns at these K).
// The lane's products and the wave sum are the workgroup form's, and the
// other waves' zero partials added there are exact, so y is the same.
constexpr int GEMV_WAVE_RW = 2;   // rows per wave
template <bool GATE, bool NT>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_wave_kernel(const GemvArgs a0, const GemvArgs a1, int nb0) {
  constexpr int RW = GEMV_WAVE_RW;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const bool second = (int)blockIdx.x >= nb0;
  const GemvArgs& a = second ? a1 : a0;
  const int blk = second ? (int)blockIdx.x - nb0 : (int)blockIdx.x;
  const int K = a.K, c = lane * 8, cc = min(c, K - 8);   // columns past K read the last chunk, times x = 0
  const int r0 = (blk * 4 + wave) * RW;
  if (r0 >= a.rows) return;   // whole wave; nothing below waits on other waves
  half8_t w[RW];
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    const half8_t* p = reinterpret_cast<const half8_t*>(a.W + (long)min(r0 + i, a.rows - 1) * a.ldw + cc);
    w[i] = NT ? __builtin_nontemporal_load(p) : *p;
  }
  float xr[8];
  if (GATE) {
    const float* src[7] = {a.gi + cc, a.gi + K + cc, a.gi + 2 * K + cc, a.gh + cc, a.gh + K + cc, a.gh + 2 * K + cc,
                           a.hp + cc};
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
      xr[j] = c < K ? (1.0f - z) * n + z * g[6][h][e] : 0.f;
    }
    if (blk == 0 && wave == 0 && c < K) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a.h1[c + j] = xr[j];
        if (a.h2) a.h2[c + j] = xr[j];
      }
    }
  } else {
    const float4_t u = *reinterpret_cast<const float4_t*>(a.x + cc);
    const float4_t v = *reinterpret_cast<const float4_t*>(a.x + cc + 4);
    const bool in = c < K;
    xr[0] = in ? u[0] : 0.f; xr[1] = in ? u[1] : 0.f; xr[2] = in ? u[2] : 0.f; xr[3] = in ? u[3] : 0.f;
    xr[4] = in ? v[0] : 0.f; xr[5] = in ? v[1] : 0.f; xr[6] = in ? v[2] : 0.f; xr[7] = in ? v[3] : 0.f;
  }
#pragma unroll
  for (int i = 0; i < RW; ++i) {
    float v = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) v = fmaf((float)w[i][j], xr[j], v);
    v = wave_sum(v);
    if (lane == i && r0 + i < a.rows) {
      if (a.bias) v += a.bias[r0 + i];
      if (a.act == GEMV_GELU) v = gelu_tanh(v);
      a.y[r0 + i] = v;
    }
  }
}

// The frame's first launch: the policy inputs (policy_inputs.h), the
// temporal GEMV and stem layer 1's im2col, which need nothing from each
// other: the GEMV reads the features where they lie in the feature ring (the
// policy inputs' features buffer is the same data, gathered), and the im2col
// reads the two sampled frames from the image ring and the staging (the
// policy inputs' image is the same data, copied).  The policy inputs write
// only ring slots of frame n, which neither reads.  Workgroups [0, npa) run
// the policy inputs, the next nblk the im2col (both short: their slots pass
// to the GEMV early; the im2col folded U blocks per workgroup, every gather
// load issued before the first store), the last nb the GEMV.
struct HeadIm2col {
  const uint8_t* warped;     // [2][6][H][W], frame n
  const uint8_t* img_ring;   // [2][img_slots][6][H][W]
  const unsigned* counter;
  half_t* patches;
  int H, W, Kp, Ho, Wo, img_slots, blocks_per_image, nblk;
};

template <int NSTEP, bool NT, int U>
__global__ __launch_bounds__(GEMV_THREADS) void frame_head_kernel(const PolicyArgs pa, int npa, const GemvArgs ga,
                                                                  int nb, const HeadIm2col c) {
  int bid = (int)blockIdx.x;
  if (bid < npa) {
    policy_inputs_at(pa, (long)bid * GEMV_THREADS + threadIdx.x);
    return;
  }
  bid -= npa;
  if (bid >= c.nblk) {
    gemv_block<NSTEP, false, NT, true>(ga, ga, nb, bid - c.nblk);
    return;
  }
  constexpr int C = 12;   // two sampled 6-channel frames
  const long n = c.counter[0];
  const int old_slot = wrap(n - (c.img_slots - 1), c.img_slots);
  const long hw = (long)c.H * c.W, fb = 6 * hw;
  const int total = 2 * c.blocks_per_image;
  const int per = c.Ho * c.Wo * (c.Kp / 8);
  half8_t v[U];
  long off[U];
  bool ok[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // clamped to the last valid block and item (their stores are dropped)
    const int j0 = bid + u * c.nblk, j = min(j0, total - 1);
    const int b = j / c.blocks_per_image;
    const int i0 = (j - b * c.blocks_per_image) * GEMV_THREADS + (int)threadIdx.x, i = min(i0, per - 1);
    const uint8_t* old_frame = c.img_ring + ((long)b * c.img_slots + old_slot) * fb;
    const uint8_t* cur_frame = c.warped + (long)b * fb;
    im2col_u8_gather_p([&](int ch) { return ch < 6 ? old_frame + ch * hw : cur_frame + (ch - 6) * hw; }, C, c.H,
                       c.W, c.Kp, c.Ho, c.Wo, b, i, v[u], off[u]);
    ok[u] = j0 < total && i0 < per;
  }
  // device-scope stores: the layer-1 conv GEMM reads the patches next
  const auto rsrc = sc1_rsrc(c.patches, 2L * 2 * c.Ho * c.Wo * c.Kp);
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
  CK_REQUIRE(a.W && a.y && (a.x || a.gi || a.xring), "gemv: null pointer");
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

int batch_rows(const GemvArgs& a) { return gemv_rows_per_wg(a.rows, a.rows_per_wg); }

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
  if (a0.K <= 512 && (!two || a1.K <= 512) && a0.rows_per_wg <= 0 && (!two || a1.rows_per_wg <= 0) && !a0.xring) {
    constexpr int per = 4 * GEMV_WAVE_RW;   // rows per workgroup
    const int nb0 = ceil_div(a0.rows, per);
    const int grid = nb0 + (two ? ceil_div(a1.rows, per) : 0);
    if (nt) CK_LAUNCH((gemv_wave_kernel<GATE, true>), dim3(grid), dim3(GEMV_THREADS), 0, s, a0, two ? a1 : a0, nb0);
    else CK_LAUNCH((gemv_wave_kernel<GATE, false>), dim3(grid), dim3(GEMV_THREADS), 0, s, a0, two ? a1 : a0, nb0);
    CK_LAUNCHED("gemv_wave");
    return;
  }
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

}  // namespace

namespace {

template <int NSTEP, bool NT>
int head_slots() {
  int dev = 0, per_cu = 0, cus = 0;
  CK_HIP(hipGetDevice(&dev));
  CK_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  CK_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &per_cu, reinterpret_cast<const void*>(frame_head_kernel<NSTEP, NT, 1>), GEMV_THREADS, 0));
  return std::max(1, per_cu) * std::max(1, cus);
}

template <int NSTEP, bool NT>
void launch_head(const PolicyArgs& pa, GemvArgs a, HeadIm2col c, int slots, hipStream_t s) {
  a.rows_per_wg = batch_rows(a);
  const int nb = ceil_div(a.rows, a.rows_per_wg);
  const int npa = ceil_div(policy_inputs_threads(pa), GEMV_THREADS);
  const long total = 2L * c.blocks_per_image;
  const long free_slots = std::max<long>((long)slots - nb - npa, ceil_div(total, 4));
  const int U = (int)std::min<long>(4, ceil_div(total, free_slots));
  c.nblk = ceil_div(total, U);
  const long grid = (long)nb + npa + c.nblk;
  CK_REQUIRE(grid < (1L << 31), "frame_head: grid too large");
  if (U == 1) CK_LAUNCH((frame_head_kernel<NSTEP, NT, 1>), dim3((unsigned)grid), dim3(GEMV_THREADS), 0, s, pa, npa, a, nb, c);
  else if (U == 2) CK_LAUNCH((frame_head_kernel<NSTEP, NT, 2>), dim3((unsigned)grid), dim3(GEMV_THREADS), 0, s, pa, npa, a, nb, c);
  else if (U == 3) CK_LAUNCH((frame_head_kernel<NSTEP, NT, 3>), dim3((unsigned)grid), dim3(GEMV_THREADS), 0, s, pa, npa, a, nb, c);
  else CK_LAUNCH((frame_head_kernel<NSTEP, NT, 4>), dim3((unsigned)grid), dim3(GEMV_THREADS), 0, s, pa, npa, a, nb, c);
  CK_LAUNCHED("frame_head");
}

template <int NSTEP>
void launch_head_nt(const PolicyArgs& pa, const GemvArgs& a, const HeadIm2col& c, bool nt, int slots, hipStream_t s) {
  if (slots <= 0) slots = nt ? head_slots<NSTEP, true>() : head_slots<NSTEP, false>();
  if (nt) launch_head<NSTEP, true>(pa, a, c, slots, s);
  else launch_head<NSTEP, false>(pa, a, c, slots, s);
}

}  // namespace

int frame_head_slots(int K, bool stream) {
  CK_REQUIRE(K > 0 && K <= 8 * GEMV_STEP_COLS, "frame_head: K must be in (0, 16384]");
  switch (ceil_div(K, GEMV_STEP_COLS)) {
    case 1: return stream ? head_slots<1, true>() : head_slots<1, false>();
    case 2: return stream ? head_slots<2, true>() : head_slots<2, false>();
    case 3: return stream ? head_slots<3, true>() : head_slots<3, false>();
    case 4: return stream ? head_slots<4, true>() : head_slots<4, false>();
    case 5: return stream ? head_slots<5, true>() : head_slots<5, false>();
    case 6: return stream ? head_slots<6, true>() : head_slots<6, false>();
    case 7: return stream ? head_slots<7, true>() : head_slots<7, false>();
    default: return stream ? head_slots<8, true>() : head_slots<8, false>();
  }
}

void launch_frame_head(const QueueDims& q, const uint8_t* warped, const float* packed, const unsigned* counter,
                       uint8_t* img_ring, float* feat_ring, float* desire_ring, uint8_t* img_out, float* feat_out,
                       float* ctx_tail, const half_t* Wt, const float* bias, float* y, int rows, int act, bool stream,
                       half_t* patches, int Kp, int slots, hipStream_t s) {
  const PolicyArgs pa =
      make_policy_args(q, warped, packed, counter, img_ring, feat_ring, desire_ring, img_out, feat_out, ctx_tail);
  const int K = q.feat_hist * q.feat_len;
  GemvArgs a = make_args(Wt, nullptr, bias, y, rows, K, K, act, 0);
  a.xring = feat_ring;
  a.xprev = packed + q.desire_len + 4;
  a.xcounter = counter;
  a.xfs = q.fs;
  a.xlen = q.feat_len;
  a.xfL = q.fs * q.feat_hist;
  check_args(a);
  CK_REQUIRE(q.feat_len % 8 == 0 && (reinterpret_cast<uintptr_t>(feat_ring) & 15) == 0 &&
                 (reinterpret_cast<uintptr_t>(a.xprev) & 15) == 0,
             "frame_head: feature rows must be whole 16-byte chunks, 16-byte aligned (feat_len % 8, desire_len % 4)");
  CK_REQUIRE(patches && Kp >= 9 * 12 && Kp % 8 == 0 && (reinterpret_cast<uintptr_t>(patches) & 15) == 0,
             "frame_head: bad im2col patches (Kp >= 108, a multiple of 8, 16-byte aligned)");
  HeadIm2col c{};
  c.warped = warped; c.img_ring = img_ring; c.counter = counter; c.patches = patches;
  c.H = q.img_h; c.W = q.img_w; c.Kp = Kp; c.img_slots = q.img_slots;
  c.Ho = (q.img_h - 1) / 2 + 1;
  c.Wo = (q.img_w - 1) / 2 + 1;
  const long per = (long)c.Ho * c.Wo * (Kp / 8);
  CK_REQUIRE(per < (1L << 30) && (long)q.img_h * q.img_w < (1L << 31), "frame_head: image too large");
  // the patches leave through raw buffer stores addressed by 32-bit offsets
  CK_REQUIRE(2L * 2 * c.Ho * c.Wo * Kp < (1L << 31), "frame_head: patch buffer must be under 2 GiB");
  c.blocks_per_image = (int)ceil_div(per, GEMV_THREADS);
  switch (ceil_div(K, GEMV_STEP_COLS)) {
    case 1: launch_head_nt<1>(pa, a, c, stream, slots, s); break;
    case 2: launch_head_nt<2>(pa, a, c, stream, slots, s); break;
    case 3: launch_head_nt<3>(pa, a, c, stream, slots, s); break;
    case 4: launch_head_nt<4>(pa, a, c, stream, slots, s); break;
    case 5: launch_head_nt<5>(pa, a, c, stream, slots, s); break;
    case 6: launch_head_nt<6>(pa, a, c, stream, slots, s); break;
    case 7: launch_head_nt<7>(pa, a, c, stream, slots, s); break;
    default: launch_head_nt<8>(pa, a, c, stream, slots, s); break;
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
