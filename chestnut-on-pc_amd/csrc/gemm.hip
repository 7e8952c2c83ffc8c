// f16-input / f32-accumulate GEMM on gfx950 MFMA: the replacement of the
// WMMA attention/projection kernels r_6_2, r_2_24, r_12_32_4, r_48_32_4
// (run_pinned2.py:100-266, 866-934; NOTES.md:84-104).
//
// Those kernels are serial K loops whose whole output tile lives in the
// register file as loop-carried fragments, one block per SM (255 registers).
// This file has two kernels instead:
//   * gemm_dma_kernel (the production path, tile codes 1-10): A and B tiles go
//     straight from global memory into an S-stage LDS ring with
//     global_load_lds_dwordx4, XOR-swizzled for conflict-free MFMA operand
//     reads; v_mfma_f32_32x32x16_f16 on a grid of 64x64 wave tiles (32x96 on
//     the 128x96 QKV tile); one or two K-groups; an LDS-staged epilogue
//     (described at the kernel);
//   * gemm_kernel (tile codes 11-14): register-staged loads with rows padded
//     to 72 halves, kept for a B operand given as [K][N], which it transposes
//     in registers.
// Both split K over extra workgroups when the output has too few tiles to
// fill 256 CUs (the graph-level split-K the reference names as its next
// lever, README.md:170-175), writing f32 partials that a reduce kernel -- or
// the LayerNorm that consumes them -- sums in split order (deterministic,
// unlike atomics); regroup tiles so each XCD's L2 holds a run of M-tiles
// sharing the same weight columns; and fuse bias / ReLU / GELU /
// residual-add / QKV-split epilogues.
// MFMA 32x32x16 operand layout (lane l of 64): A row l%32, k = 8*(l/32)..+7;
// B column l%32, same k; D element e of lane l is row 8*(e/4) + 4*(l/32) +
// e%4, column l%32.  The layout is checked by the MFMA KAT (wmma.hip).
#include <mutex>
#include <type_traits>
#include <utility>
#include <vector>

#include "common.h"
#include "gemv_block.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr int BK = 64;
// LDS ring stages of the LDS-DMA kernel's two-K-group configurations, and
// whether the f32 staging of both groups (8 regions of (BM/2) x (BN/2 + 8)
// floats) fits in that ring.
constexpr int dma_stages_kg2(int BM, int BN) {
  return (BM == 64 && BN == 64) ? 4 : (6 * (BM + BN) * BK * 2 <= 163840 ? 6 : 4);
}
constexpr bool kg2_staging_fits(int BM, int BN, int S) { return 2 * 4 * (BM / 2) * (BN / 2 + 8) * 4 <= S * (BM + BN) * BK * 2; }
constexpr int LDK = BK + 8;   // padded LDS row (halves)

struct GemmParams {
  const half_t* A;
  const half_t* B;
  void* C;
  const float* bias;
  float* ws;
  half_t* vt;
  long lda, ldb, ldc, vt_ld;
  long sA, sB, sC, sBias;
  int M, N, K, kps;   // kps: K per split
  int split, batch, Mt, Nt;
  int qk_cols;
  int head_dim;       // EPI_QKV_FRAG
  int vec;            // 1: shapes/alignment allow the LDS-staged 16-byte epilogue
  const half_t* pos;  // EPI_EMBED
  const float* ctx;   // EPI_EMBED
  int cc_log2, ch, cw, cwo;   // implicit conv: log2(channels), input height/width, output width
  const half_t* zero;         // implicit conv: 16 zero bytes
  int c_nm;                   // the split-K reduce stores element (m, n) at C[n*ldc + m]
  unsigned* pair;             // split 2, f32 output: ticket counters of the in-kernel finish (null: a reduce follows)
};

// Implicit 3x3 stride-2 pad-1 convolution: the A chunk (8 halves) of patch
// row m, columns k .. k+7 (one tap, 8 channels: C >= 8) is input pixel
// (2*ho - 1 + tap/3, 2*wo - 1 + tap%3), channels k%C .. +7, or zeros outside
// the image and beyond the 9 taps.  yb/xb: 2*ho - 1, 2*wo - 1 of the row.
__device__ __forceinline__ const half_t* conv_a_src(const GemmParams& p, const half_t* img, int yb, int xb, int k) {
  const int tap = k >> p.cc_log2, c = k & ((1 << p.cc_log2) - 1);
  const int dy = (tap * 11) >> 5;   // tap / 3 for tap < 9
  const int y = yb + dy, x = xb + tap - 3 * dy;
  const bool ok = tap < 9 && (unsigned)y < (unsigned)p.ch && (unsigned)x < (unsigned)p.cw;
  return ok ? img + (((long)y * p.cw + x) << p.cc_log2) + c : p.zero;
}

template <int EPI>
__device__ __forceinline__ void epi_store(const GemmParams& p, void* C, const float* bias, int m, int n, float v) {
  if (EPI == EPI_F32) {
    if (bias) v += bias[n];
    static_cast<float*>(C)[(long)m * p.ldc + n] = v;
  } else if (EPI == EPI_EMBED) {
    if (bias) v += bias[n];
    static_cast<float*>(C)[(long)m * p.ldc + n] = v + ((float)p.pos[(long)m * p.ldc + n] + p.ctx[n]);
  } else if (EPI == EPI_F32_RESID) {
    if (bias) v += bias[n];
    float* c = static_cast<float*>(C) + (long)m * p.ldc + n;
    *c = *c + v;
  } else {
    if (bias) v += bias[n];
    if (EPI == EPI_F16_BIAS_RELU) v = fmaxf(v, 0.f);
    if (EPI == EPI_F16_BIAS_GELU) v = gelu_fast(v);
    if (EPI == EPI_QKV_FRAG) {
      return;   // unreachable: the host admits EPI_QKV_FRAG only with the staged epilogue
    } else if (EPI == EPI_QKV && n >= p.qk_cols) {
      p.vt[(long)(n - p.qk_cols) * p.vt_ld + m] = (half_t)v;
    } else if (p.c_nm) {
      static_cast<half_t*>(C)[(long)n * p.ldc + m] = (half_t)v;
    } else {
      static_cast<half_t*>(C)[(long)m * p.ldc + n] = (half_t)v;
    }
  }
}

// 8x8 transpose of f16 values held as 8 rows of 4 packed words.
__device__ __forceinline__ void transpose8x8(const uint32_t (&in)[8][4], uint32_t (&out)[8][4]) {
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = in[2 * j][q], b = in[2 * j + 1][q];
      out[2 * q][j] = (a & 0xFFFFu) | (b << 16);            // column 2q: low halves
      out[2 * q + 1][j] = (a >> 16) | (b & 0xFFFF0000u);    // column 2q+1: high halves
    }
  }
}

template <int BM, int BN, bool BKN, int EPI>
__global__ __launch_bounds__(256) void gemm_kernel(const GemmParams p) {
  __shared__ __attribute__((aligned(16))) half_t As[2][BM][LDK];
  __shared__ __attribute__((aligned(16))) half_t Bs[2][BN][LDK];

  constexpr int WM = BM / 2, WN = BN / 2;   // wave sub-tile
  constexpr int FM = WM / 32, FN = WN / 32;
  constexpr int ACH = BM * BK / 8 / 256;    // 16-byte A chunks per thread
  constexpr int BCH = BN * BK / 8 / 256;    // 16-byte B chunks per thread (NK layout)

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // ---- tile decode (XCD-grouped) ----
  const int total = p.Mt * p.Nt * p.split * p.batch;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int mt = L % p.Mt; L /= p.Mt;
  const int nt = L % p.Nt; L /= p.Nt;
  const int sp = L % p.split;
  const int bz = L / p.split;

  const half_t* A = p.A + bz * p.sA;
  const half_t* B = p.B + bz * p.sB;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = sp * p.kps;
  const int nk = p.kps / BK;

  // ---- global -> register loaders ----
  half8_t ra[ACH];
  half8_t rb[BKN ? 8 : BCH];
  auto load_tiles = [&](int k0) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, row = c >> 3, kc = (c & 7) * 8;
      const int gm = min(m0 + row, p.M - 1);
      ra[i] = *reinterpret_cast<const half8_t*>(A + (long)gm * p.lda + k0 + kc);
    }
    if (!BKN) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + 256 * i, row = c >> 3, kc = (c & 7) * 8;
        const int gn = min(n0 + row, p.N - 1);
        rb[i] = *reinterpret_cast<const half8_t*>(B + (long)gn * p.ldb + k0 + kc);
      }
    } else if (tid < BN) {
      // B is [K][N]: thread loads an 8(k) x 8(n) block, transposed on store
      const int kb = tid / (BN / 8), nb = tid % (BN / 8);
      const int gn = min(n0 + nb * 8, p.N - 8);
#pragma unroll
      for (int r = 0; r < 8; ++r)
        rb[r] = *reinterpret_cast<const half8_t*>(B + (long)(k0 + kb * 8 + r) * p.ldb + gn);
    }
  };
  auto store_tiles = [&](int buf) {
#pragma unroll
    for (int i = 0; i < ACH; ++i) {
      const int c = tid + 256 * i, row = c >> 3, kc = (c & 7) * 8;
      *reinterpret_cast<half8_t*>(&As[buf][row][kc]) = ra[i];
    }
    if (!BKN) {
#pragma unroll
      for (int i = 0; i < BCH; ++i) {
        const int c = tid + 256 * i, row = c >> 3, kc = (c & 7) * 8;
        *reinterpret_cast<half8_t*>(&Bs[buf][row][kc]) = rb[i];
      }
    } else if (tid < BN) {
      const int kb = tid / (BN / 8), nb = tid % (BN / 8);
      uint32_t in[8][4], out[8][4];
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        const uint32_t* w = reinterpret_cast<const uint32_t*>(&rb[r]);
#pragma unroll
        for (int q = 0; q < 4; ++q) in[r][q] = w[q];
      }
      transpose8x8(in, out);
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(&Bs[buf][nb * 8 + c][kb * 8]);
        dst[0] = out[c][0]; dst[1] = out[c][1]; dst[2] = out[c][2]; dst[3] = out[c][3];
      }
    }
  };

  float16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float16_t{};

  load_tiles(kbeg);
  store_tiles(0);
  __syncthreads();

  for (int it = 0; it < nk; ++it) {
    const int buf = it & 1;
    if (it + 1 < nk) load_tiles(kbeg + (it + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 16) {
      half8_t af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const half8_t*>(&As[buf][wm * WM + i * 32 + (lane & 31)][kk + (lane >> 5) * 8]);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bf[j] = *reinterpret_cast<const half8_t*>(&Bs[buf][wn * WN + j * 32 + (lane & 31)][kk + (lane >> 5) * 8]);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (it + 1 < nk) {
      store_tiles(buf ^ 1);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  if (p.split > 1 || EPI == EPI_PARTIALS) {
    float* ws = p.ws + ((long)sp * p.batch + bz) * (long)p.M * p.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
          const int n = n0 + wn * WN + j * 32 + (lane & 31);
          if (m < p.M && n < p.N) ws[(long)m * p.N + n] = acc[i][j][e];
        }
    return;
  }
  void* C = (EPI == EPI_F32 || EPI == EPI_F32_RESID || EPI == EPI_EMBED)
                ? static_cast<void*>(static_cast<float*>(p.C) + bz * p.sC)
                : static_cast<void*>(static_cast<half_t*>(p.C) + bz * p.sC);
  const float* bias = p.bias ? p.bias + bz * p.sBias : nullptr;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * WM + i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        const int n = n0 + wn * WN + j * 32 + (lane & 31);
        if (m < p.M && n < p.N) epi_store<EPI>(p, C, bias, m, n, acc[i][j][e]);
      }
}

// Sums split-K partials in split order, then applies the epilogue.  With
// N % 4 == 0 a thread owns 4 consecutive outputs of one row (16-byte partial
// loads); the partials of up to 8 splits are loaded before they are added.
// Thread t of the split-K reduce: output elements t*per .. t*per+per-1.
template <int EPI>
__device__ __forceinline__ void splitk_reduce_at(const GemmParams& p, long t) {
  const long MN = (long)p.M * p.N;
  const bool v4 = (p.N & 3) == 0;
  const int per = v4 ? 4 : 1;
  const long idx = t * per;
  if (idx >= MN * p.batch) return;
  const int bz = (int)(idx / MN);
  const long r = idx - bz * MN;
  const int m = (int)(r / p.N), n = (int)(r - (long)m * p.N);
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < p.split; s0 += 8) {
    float4_t part[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float* src = p.ws + ((long)(s0 + i) * p.batch + bz) * MN + r;
      if (s0 + i >= p.split) part[i] = float4_t{0.f, 0.f, 0.f, 0.f};
      else if (v4) part[i] = *reinterpret_cast<const float4_t*>(src);
      else part[i] = float4_t{*src, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (s0 + i < p.split)
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += part[i][e];
  }
  void* C = (EPI == EPI_F32 || EPI == EPI_F32_RESID || EPI == EPI_EMBED)
                ? static_cast<void*>(static_cast<float*>(p.C) + bz * p.sC)
                : static_cast<void*>(static_cast<half_t*>(p.C) + bz * p.sC);
  const float* bias = p.bias ? p.bias + bz * p.sBias : nullptr;
  // Row-major outputs take the thread's 4 values in one 16-byte (f32) or
  // 8-byte (f16) store where the address allows: the same values as
  // epi_store, a quarter of the store instructions.
  if (v4 && (EPI == EPI_F32 || ((EPI == EPI_F16_BIAS || EPI == EPI_F16_BIAS_RELU || EPI == EPI_F16_BIAS_GELU) &&
                                !p.c_nm))) {
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = bias ? v[e] + bias[n + e] : v[e];
      if (EPI == EPI_F16_BIAS_RELU) o[e] = fmaxf(o[e], 0.f);
      if (EPI == EPI_F16_BIAS_GELU) o[e] = gelu_fast(o[e]);
    }
    if (EPI == EPI_F32) {
      float* c = static_cast<float*>(C) + (long)m * p.ldc + n;
      if ((reinterpret_cast<uintptr_t>(c) & 15) == 0) {
        *reinterpret_cast<float4_t*>(c) = float4_t{o[0], o[1], o[2], o[3]};
        return;
      }
    } else {
      half_t* c = static_cast<half_t*>(C) + (long)m * p.ldc + n;
      if ((reinterpret_cast<uintptr_t>(c) & 7) == 0) {
        *reinterpret_cast<half4_t*>(c) = half4_t{(half_t)o[0], (half_t)o[1], (half_t)o[2], (half_t)o[3]};
        return;
      }
    }
  }
  for (int e = 0; e < per; ++e) epi_store<EPI>(p, C, bias, m, n + e, v[e]);
}

template <int EPI>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmParams p) {
  splitk_reduce_at<EPI>(p, (long)blockIdx.x * 256 + threadIdx.x);
}

// The split-K reduce with an independent GEMV riding along: workgroups
// [0, nr) reduce, the rest run the GEMV (gemv_block.h), so a small product
// the frame needs anyway costs no launch of its own.
template <int EPI, int NSTEP, bool NT>
__global__ __launch_bounds__(256) void splitk_reduce_gemv_kernel(const GemmParams p, int nr, const GemvArgs g,
                                                                 int nb) {
  if ((int)blockIdx.x < nr) {
    splitk_reduce_at<EPI>(p, (long)blockIdx.x * 256 + threadIdx.x);
    return;
  }
  gemv_block<NSTEP, false, NT>(g, g, nb, (int)blockIdx.x - nr);
}

// ---------------------------------------------------------------------------
// NT GEMM with direct global->LDS loads (gfx950 global_load_lds_dwordx4) into
// an S-stage LDS ring, issued S-1 K-steps ahead of the MFMAs.
//
// * No staging registers and no ds_write: each load instruction of a wave
//   deposits 64 lanes x 16 bytes = 8 tile rows x 128 bytes contiguously.
// * LDS rows (128 bytes) are stored XOR-swizzled by 16-byte chunk: physical
//   chunk p of row r holds logical chunk p ^ ((r >> 1) & 7).  The LDS serves
//   16 lanes x 16 bytes per cycle over 64 banks; two consecutive rows fill the
//   256-byte bank window, and the swizzle gives the 8 even (odd) rows of any
//   16 consecutive ones 8 distinct chunk positions, so the MFMA operand reads
//   are conflict free.  The swizzle is applied through the global addresses
//   each lane fetches.
// * One barrier per K-step: each wave waits (vmcnt) only for its own loads of
//   the step about to be consumed, then the barrier publishes every wave's
//   loads and retires the previous step's readers, whose stage is refilled.
//   The barrier is the raw s_barrier: the release fence of __syncthreads
//   would drain vmcnt to zero on gfx9 and serialise the prefetch.
// ---------------------------------------------------------------------------

// Issue one K-step's loads of this wave into LDS stage `st` (A rows then B rows).
// ko: the K-step's offset in A (halves); bko: in B (ko for a [N][K] B, ko
// rows of ldb for a [K][N] B).  BPOL: the B loads' cache policy (0, or 2 =
// non-temporal, see gemm_dma_kernel).
template <int NIA, int NIB, int STAGE_A, int BPOL = 0>
__device__ __forceinline__ void dma_issue(const half_t* const* asrc, const half_t* const* bsrc, half_t* st, int wave,
                                          int ko, long bko) {
#pragma unroll
  for (int i = 0; i < NIA; ++i)
    __builtin_amdgcn_global_load_lds(asrc[i] + ko, (lds_ptr_t)(st + (wave * NIA + i) * 8 * BK), 16, 0, 0);
#pragma unroll
  for (int i = 0; i < NIB; ++i)
    __builtin_amdgcn_global_load_lds(bsrc[i] + bko, (lds_ptr_t)(st + STAGE_A + (wave * NIB + i) * 8 * BK), 16, 0,
                                     BPOL);
}

// Coalesced epilogue.  The MFMA accumulator layout gives a lane one column
// and scattered rows, so direct stores are 2- or 4-byte pieces spread over
// 32 rows per instruction (and, for the transposed V of the QKV epilogue,
// over 32 V^T rows).  Instead each wave puts its finished (WM x WN) sub-tile
// -- bias and activation applied, converted to the output type -- into a
// private LDS region and writes it out as whole 16-byte row chunks.  V
// columns are staged transposed ([n][m]), four consecutive rows of a lane
// forming one 8-byte LDS write, so V^T rows leave contiguously as well.
// Row pitches carry 16 bytes of padding so the two half-waves' staging
// writes (rows r and r+4) fall in different banks.  Every staged output --
// split-K partials, f32 outputs (plain, residual-add, embedding), row-major
// f16 outputs and the QKV fragments, all read by the next kernel -- leaves
// with the device-scope cache policy (store_sc1: -0.5%, -0.4% and -0.3% of
// the 1B frame for the partials, the f16 outputs and the fragments against
// non-temporal or default stores) wherever the region is addressable by a
// 32-bit buffer offset (sc1_ok), and with non-temporal stores otherwise.
// Requires (checked on the host, else the direct per-element stores run):
// N % 8 == 0, ldc / batch stride / base of C and ws 16-byte compatible,
// and for QKV qk_cols % BN == 0 (% 32 on the 128x96 tile), M % 8 == 0 and
// vt_ld % 8 == 0.
//
// EPI_QKV_FRAG writes the attention kernel's MFMA operands directly, in
// 16-byte chunks ordered so that one wave's fragment load is one contiguous
// KB (16 lanes x 16 B per row of the fragment would otherwise touch 16
// separate rows).  With T = M tokens, d = qk_cols / 2, hd = head_dim,
// H = d / hd, chunk c of a fragment holds 8 halves for lane l = 16*g + r:
//   Q, K (16x16x32 A/B operand: row r = token, 8 head dims from 8*g):
//     C chunk (((w*H + h) * T/16 + t/16) * hd/32 + j/32) * 64 + 16*((j%32)/8) + t%16
//     for token t, head dim j of head h; w = 0 for Q, 1 for K.
//   V (B operand of P.V: column r = head dim, tokens 4g..4g+3 and
//   16+4g..16+4g+3 of a 32-token block, the attention kernel's key order):
//     vt chunk ((h * hd/16 + j/16) * T/32 + t/32) * 64 + 16*((t%16)/4) + j%16,
//     element (t/16)*4 + t%4 of the chunk.
// SWP (every epilogue but the QKV ones): the accumulators hold D^T (the MFMA
// ran with its operands swapped), so element e of tile (i, j) is row
// i*32 + lane%32, column j*32 + 8*(e/4) + 4*(lane/32) + e%4: a lane's four
// consecutive e are four consecutive columns of one row, staged with one 8-
// or 16-byte LDS write instead of four scalar ones; bcol[j][e] is the bias
// of that column (bcol[j][0] of column j*32 + lane%32 otherwise).
template <int WM, int WN, int FM, int FN, int EPI, bool SWP, int NBC>
__device__ __forceinline__ void store_staged(const GemmParams& p, const float16_t (&acc)[FM][FN],
                                             const float (&bcol)[FN][NBC], char* region, int mw, int nw, int sp,
                                             int bz, int lane) {
  const bool to_ws = p.split > 1 || EPI == EPI_PARTIALS;
  if (to_ws || EPI == EPI_F32 || EPI == EPI_F32_RESID || EPI == EPI_EMBED) {
    constexpr int PF = WN + 8;   // floats
    float* st = reinterpret_cast<float*>(region);
    if constexpr (SWP) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            float4_t v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * k + e] + bcol[j][4 * k + e];
            *reinterpret_cast<float4_t*>(st + (i * 32 + (lane & 31)) * PF + j * 32 + 8 * k + 4 * (lane >> 5)) = v;
          }
    } else {
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int c = j * 32 + (lane & 31);
        const float bv = bcol[j][0];
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int e = 0; e < 16; ++e)
            st[(i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * PF + c] = acc[i][j][e] + bv;
      }
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    constexpr int CPR = WN / 4;   // 16-byte chunks per row
    float* dst = to_ws ? p.ws + ((long)sp * p.batch + bz) * (long)p.M * p.N : static_cast<float*>(p.C) + bz * p.sC;
    const long ld = to_ws ? p.N : p.ldc;
    const long plane = to_ws ? 4L * p.M * p.N : 4L * ((long)(p.M - 1) * p.ldc + p.N);
    const bool sc1 = sc1_ok(plane);
    const __amdgpu_buffer_rsrc_t rs = sc1_rsrc(dst, sc1 ? plane : 0);
#pragma unroll 4
    for (int q = lane; q < WM * CPR; q += 64) {
      const int r = q / CPR, c = (q % CPR) * 4;
      const int m = mw + r, n = nw + c;
      if (m >= p.M || n >= p.N) continue;
      float4_t v = *reinterpret_cast<const float4_t*>(st + r * PF + c);
      float4_t* g = reinterpret_cast<float4_t*>(dst + (long)m * ld + n);
      if (!to_ws && EPI == EPI_F32_RESID) v += *g;
      if (!to_ws && EPI == EPI_EMBED) {
        const half4_t ps = *reinterpret_cast<const half4_t*>(p.pos + (long)m * p.ldc + n);
        const float4_t cs = *reinterpret_cast<const float4_t*>(p.ctx + n);
        v += float4_t{(float)ps[0] + cs[0], (float)ps[1] + cs[1], (float)ps[2] + cs[2], (float)ps[3] + cs[3]};
      }
      if (sc1) store_sc1(rs, ((long)m * ld + n) * 4, v);
      else __builtin_nontemporal_store(v, g);
    }
    return;
  }
  half_t* st = reinterpret_cast<half_t*>(region);
  if ((EPI == EPI_QKV || EPI == EPI_QKV_FRAG) && nw >= p.qk_cols) {
    constexpr int PT = WM + 8;   // halves, transposed rows [n][m]
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int c = j * 32 + (lane & 31);
      const float bv = bcol[j][0];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          half4_t h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (half_t)(acc[i][j][4 * g4 + e] + bv);
          *reinterpret_cast<half4_t*>(st + c * PT + i * 32 + 8 * g4 + 4 * (lane >> 5)) = h;
        }
    }
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
    if (EPI == EPI_QKV_FRAG) {
      // V fragment blocks: 16 features x 32 tokens = 64 lanes x 8 tokens, one
      // contiguous KB per block (see the layout note at the epilogue modes)
      // The wave's WN columns lie in one head (head_dim is a power of two >= WN,
      // checked on the host), so the head and the first 16-feature block are
      // wave-uniform and the chunk index is shifts and adds.
      const int r = lane & 15, g = lane >> 4, hs = __builtin_ctz(p.head_dim);
      const int f0 = nw - p.qk_cols, h = f0 >> hs, c0 = f0 & (p.head_dim - 1);
      const long cbase = (long)(h << (hs - 4)) + (c0 >> 4);   // 16-feature block of the wave's first column
      const int tpb = p.M >> 5;                                 // 32-token blocks
#pragma unroll
      for (int blk = 0; blk < (WN / 16) * (WM / 32); ++blk) {
        const int cb = blk % (WN / 16), tb = blk / (WN / 16);
        if (mw + tb * 32 >= p.M) continue;
        // tokens 4g..4g+3 and 16+4g..16+4g+3 of the 32-token block: the key
        // order in which the attention kernel's P.V A operand leaves its softmax
        const int nl = cb * 16 + r, ml = tb * 32 + g * 4;
        const long chunk = ((cbase + cb) * tpb + (mw >> 5) + tb) * 64 + g * 16 + r;
        const half4_t lo = *reinterpret_cast<const half4_t*>(st + nl * PT + ml);
        const half4_t hi = *reinterpret_cast<const half4_t*>(st + nl * PT + ml + 16);
        store_sc1(sc1_rsrc(p.vt, 2L * p.M * (p.N - p.qk_cols)), chunk * 16,
                  half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
      }
      return;
    }
    constexpr int CPR = WM / 8;
#pragma unroll 4
    for (int q = lane; q < WN * CPR; q += 64) {
      const int r = q / CPR, c = (q % CPR) * 8;
      const int n = nw + r, m = mw + c;
      if (n >= p.N || m >= p.M) continue;
      *reinterpret_cast<half8_t*>(p.vt + (long)(n - p.qk_cols) * p.vt_ld + m) =
          *reinterpret_cast<const half8_t*>(st + r * PT + c);
    }
    return;
  }
  constexpr int PH = WN + 8;   // halves
  if constexpr (SWP) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          half4_t hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = acc[i][j][4 * k + e] + bcol[j][4 * k + e];
            if (EPI == EPI_F16_BIAS_RELU) v = fmaxf(v, 0.f);
            if (EPI == EPI_F16_BIAS_GELU) v = gelu_fast(v);
            hv[e] = (half_t)v;
          }
          *reinterpret_cast<half4_t*>(st + (i * 32 + (lane & 31)) * PH + j * 32 + 8 * k + 4 * (lane >> 5)) = hv;
        }
  } else {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int c = j * 32 + (lane & 31);
      const float bv = bcol[j][0];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float v = acc[i][j][e] + bv;
          if (EPI == EPI_F16_BIAS_RELU) v = fmaxf(v, 0.f);
          if (EPI == EPI_F16_BIAS_GELU) v = gelu_fast(v);
          st[(i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * PH + c] = (half_t)v;
        }
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  if (EPI == EPI_QKV_FRAG) {
    // Q / K fragment blocks: 16 tokens x 32 features = 64 lanes x 8 features
    // Q or K, the head and the first 32-feature block are wave-uniform (the
    // wave's WN columns lie in one head, as for V above).
    const int r = lane & 15, g = lane >> 4, hs = __builtin_ctz(p.head_dim), dh = p.qk_cols >> 1;
    const int which = nw >= dh, f0 = nw - which * dh, h = f0 >> hs, c0 = f0 & (p.head_dim - 1);
    const long hbase = (long)(which * (dh >> hs) + h) * (p.M >> 4);   // 16-token blocks before this head
    const int kpb = p.head_dim >> 5;                                  // 32-feature blocks per head
#pragma unroll
    for (int blk = 0; blk < (WM / 16) * (WN / 32); ++blk) {
      const int tb = blk % (WM / 16), kb = blk / (WM / 16);
      if (mw + tb * 16 >= p.M) continue;
      const int ml = tb * 16 + r, nl = kb * 32 + g * 8;
      const long chunk = ((hbase + (mw >> 4) + tb) * kpb + (c0 >> 5) + kb) * 64 + g * 16 + r;
      store_sc1(sc1_rsrc(p.C, 2L * p.M * p.qk_cols), chunk * 16, *reinterpret_cast<const half8_t*>(st + ml * PH + nl));
    }
    return;
  }
  constexpr int CPR = WN / 8;
  half_t* dst = static_cast<half_t*>(p.C) + bz * p.sC;
  const long span = 2L * ((long)(p.M - 1) * p.ldc + p.N);   // bytes of this batch's output
  const bool sc1 = sc1_ok(span);
  const __amdgpu_buffer_rsrc_t rs = sc1_rsrc(dst, sc1 ? span : 0);
#pragma unroll 4
  for (int q = lane; q < WM * CPR; q += 64) {
    const int r = q / CPR, c = (q % CPR) * 8;
    const int m = mw + r, n = nw + c;
    if (m >= p.M || n >= p.N) continue;
    const half8_t v = *reinterpret_cast<const half8_t*>(st + r * PH + c);
    if (sc1) store_sc1(rs, ((long)m * p.ldc + n) * 2, v);
    else __builtin_nontemporal_store(v, reinterpret_cast<half8_t*>(dst + (long)m * p.ldc + n));
  }
}

// The QKV fragment epilogue for waves whose columns may straddle a head or
// the Q/K/V boundaries (the 128x96 tile: one wave per 32 rows, 96 columns).
// Each 32-column block of the wave is handled on its own; its kind (Q/K or
// V), head and feature block are wave-uniform per block, and its chunks are
// the ones store_staged writes for it: Q/K blocks are staged row-major
// ([m][n], pitch WN + 8 halves) and V blocks transposed ([n][m], pitch
// WM + 8) in two areas of the wave's LDS region.
template <int WM, int WN, int FM, int FN>
__device__ __forceinline__ void store_qkv_frag_blocks(const GemmParams& p, const float16_t (&acc)[FM][FN],
                                                      const float (&bcol)[FN][1], char* region, int mw, int nw,
                                                      int lane) {
  constexpr int PH = WN + 8, PT = WM + 8;
  half_t* sq = reinterpret_cast<half_t*>(region);   // [WM][PH]
  half_t* sv = sq + WM * PH;                          // [WN][PT]
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int c = j * 32 + (lane & 31);
    const float bv = bcol[j][0];
    if (nw + j * 32 >= p.qk_cols) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          half4_t h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (half_t)(acc[i][j][4 * g4 + e] + bv);
          *reinterpret_cast<half4_t*>(sv + c * PT + i * 32 + 8 * g4 + 4 * (lane >> 5)) = h;
        }
    } else {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          sq[(i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * PH + c] = (half_t)(acc[i][j][e] + bv);
    }
  }
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  const int r = lane & 15, g = lane >> 4, hs = __builtin_ctz(p.head_dim), dh = p.qk_cols >> 1;
  const auto rq = sc1_rsrc(p.C, 2L * p.M * p.qk_cols);
  const auto rv = sc1_rsrc(p.vt, 2L * p.M * (p.N - p.qk_cols));
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int f = nw + j * 32;   // the block's first column
    if (f >= p.N) continue;
    if (f >= p.qk_cols) {
      // V: per 32-token slice two blocks of 16 features x 32 tokens
      const int f0 = f - p.qk_cols, h = f0 >> hs, c0 = f0 & (p.head_dim - 1);
      const long cbase = (long)(h << (hs - 4)) + (c0 >> 4);
      const int tpb = p.M >> 5;
#pragma unroll
      for (int blk = 0; blk < 2 * (WM / 32); ++blk) {
        const int cb = blk & 1, tb = blk >> 1;
        if (mw + tb * 32 >= p.M) continue;
        const int nl = j * 32 + cb * 16 + r, ml = tb * 32 + g * 4;
        const long chunk = ((cbase + cb) * tpb + (mw >> 5) + tb) * 64 + g * 16 + r;
        const half4_t lo = *reinterpret_cast<const half4_t*>(sv + nl * PT + ml);
        const half4_t hi = *reinterpret_cast<const half4_t*>(sv + nl * PT + ml + 16);
        store_sc1(rv, chunk * 16, half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
      }
    } else {
      // Q or K: blocks of 16 tokens x 32 features
      const int which = f >= dh, f0 = f - which * dh, h = f0 >> hs, c0 = f0 & (p.head_dim - 1);
      const long hbase = (long)(which * (dh >> hs) + h) * (p.M >> 4);   // 16-token blocks before this head
      const int kpb = p.head_dim >> 5;
#pragma unroll
      for (int tb = 0; tb < WM / 16; ++tb) {
        if (mw + tb * 16 >= p.M) continue;
        const int ml = tb * 16 + r, nl = j * 32 + g * 8;
        const long chunk = ((hbase + (mw >> 4) + tb) * kpb + (c0 >> 5)) * 64 + g * 16 + r;
        store_sc1(rq, chunk * 16, *reinterpret_cast<const half8_t*>(sq + ml * PH + nl));
      }
    }
  }
}

// Issue the load instructions [lo, hi) of a K-step (A rows first, then B
// rows); lo and hi are compile-time after unrolling, so the untaken ones vanish.
template <int NIA, int NIB, int STAGE_A, int BPOL = 0>
__device__ __forceinline__ void dma_issue_range(const half_t* const* asrc, const half_t* const* bsrc, half_t* st,
                                                int wave, int ko, long bko, int lo, int hi) {
#pragma unroll
  for (int i = 0; i < NIA; ++i)
    if (i >= lo && i < hi)
      __builtin_amdgcn_global_load_lds(asrc[i] + ko, (lds_ptr_t)(st + (wave * NIA + i) * 8 * BK), 16, 0, 0);
#pragma unroll
  for (int i = 0; i < NIB; ++i)
    if (NIA + i >= lo && NIA + i < hi)
      __builtin_amdgcn_global_load_lds(bsrc[i] + bko, (lds_ptr_t)(st + STAGE_A + (wave * NIB + i) * 8 * BK), 16, 0,
                                       BPOL);
}

// Swizzle of a [K][N] B stage (rows of 128 halves = 16 chunks of 16 bytes):
// physical chunk = logical chunk ^ bt_swz(row).  The 64 lanes of one
// transposed fragment read cover rows r0..r0+3 and r0+8..r0+11 (r0 a multiple
// of 4) x 4 chunks; the swizzle sends them to 16 distinct chunks, two lanes'
// 8 bytes per chunk, the fewest passes 512 bytes take.
__device__ __forceinline__ int bt_swz(int row) { return ((row & 3) << 2) | ((row >> 3) & 1); }

// Split-K in pairs (split 2, f32 output, p.pair set; the staged two-group
// epilogue): the two waves that computed the same rows of a sub-tile over
// the two halves of K finish them between them, with no reduce launch.  Each
// has stored its partial rows with device-scope (sc1) stores; it waits until
// they have completed, then takes a ticket, an atomic add on the rows'
// counter.  Every launch adds exactly two to each counter it uses, so the
// counters are even between launches and an odd ticket marks the second wave
// of the pair.  That wave reads the other split's rows with device-scope
// loads (the other wave's stores had completed before its ticket, which
// this wave has seen) and writes C = (0 + own) + other (+ bias): the value the
// reduce computes, (0 + p0) + p1 (+ bias), since a sum of two floats does not
// depend on their order, the sign of a zero included.  No wave waits for
// another.  own[i]: the wave's partial chunk i (row r0 + q / CPR, column
// nw + 4 (q % CPR), q = lane + 64 i); tix: the rows' counter.
template <int NQ, int HR, int CPR>
__device__ __forceinline__ void pair_finish(const GemmParams& p, const float4_t (&own)[NQ], int r0, int nw, int sp,
                                            int bz, int tix, int lane) {
  asm volatile("" ::: "memory");
  wait_vm_lgkm0<0>();   // this wave's partial stores have completed at device scope
  asm volatile("" ::: "memory");
  unsigned tk = 0;
  if (lane == 0) tk = __hip_atomic_fetch_add(p.pair + tix, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  tk = __builtin_amdgcn_readfirstlane(tk);
  asm volatile("" ::: "memory");
  if ((tk & 1u) == 0) return;   // first of the pair: the other wave finishes these rows
  const long MN = (long)p.M * p.N;
  const __amdgpu_buffer_rsrc_t ro = sc1_rsrc(p.ws + ((long)(1 - sp) * p.batch + bz) * MN, 4 * MN);
  float4_t o[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = lane + 64 * i, m = r0 + q / CPR, n = nw + (q % CPR) * 4;
    o[i] = (m < p.M && n < p.N) ? load_sc1_f4(ro, ((long)m * p.N + n) * 4) : float4_t{0.f, 0.f, 0.f, 0.f};
  }
  float* C = static_cast<float*>(p.C) + bz * p.sC;
  const float* bias = p.bias ? p.bias + bz * p.sBias : nullptr;
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = lane + 64 * i, m = r0 + q / CPR, n = nw + (q % CPR) * 4;
    if (m >= p.M || n >= p.N) continue;
    float4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = (0.f + own[i][e]) + o[i][e];
      if (bias) v[e] += bias[n + e];
    }
    *reinterpret_cast<float4_t*>(C + (long)m * p.ldc + n) = v;
  }
}

// The two K-groups' sum fused into the staged f32 epilogue (EPI_F32 and
// EPI_PARTIALS on kernels with two K-groups of NWG waves): every wave stages
// its group's sub-tile in a region of its own (group g, wave w: region
// g * NWG + w), one barrier, then the two waves of sub-tile w write half of
// its rows each, as 16-byte chunks of group 0 + group 1 (+ bias) -- the sum
// the LDS hand-over forms (group 0's accumulators += group 1's) with one
// barrier fewer, no 4-byte LDS traffic and the stores spread over both
// groups.  Called by all 2 * NWG waves after their last ring read has
// retired (barrier); base: the LDS ring.
template <int WM, int WN, int FM, int FN, int EPI, bool SWP, int NWG>
__device__ __forceinline__ void store_staged_kg2(const GemmParams& p, const float16_t (&acc)[FM][FN], char* base,
                                                 int grp, int w4, int mw, int nw, int sp, int bz, int tile, int lane) {
  static_assert(EPI == EPI_F32 || EPI == EPI_PARTIALS, "f32 outputs only");
  constexpr int PF = WN + 8, REGION = WM * PF * 4, CPR = WN / 4;
  float* st = reinterpret_cast<float*>(base + (grp * NWG + w4) * REGION);
  if constexpr (SWP) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          float4_t v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = acc[i][j][4 * k + e];
          *reinterpret_cast<float4_t*>(st + (i * 32 + (lane & 31)) * PF + j * 32 + 8 * k + 4 * (lane >> 5)) = v;
        }
  } else {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e)
          st[(i * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3)) * PF + j * 32 + (lane & 31)] = acc[i][j][e];
  }
  wait_vm_lgkm0<0>();
  lds_barrier();
  const float* s0 = reinterpret_cast<const float*>(base + w4 * REGION);
  const float* s1 = reinterpret_cast<const float*>(base + (NWG + w4) * REGION);
  const bool to_ws = p.split > 1 || EPI == EPI_PARTIALS;
  float* dst = to_ws ? p.ws + ((long)sp * p.batch + bz) * (long)p.M * p.N : static_cast<float*>(p.C) + bz * p.sC;
  const long ld = to_ws ? p.N : p.ldc;
  const long plane = to_ws ? 4L * p.M * p.N : 4L * ((long)(p.M - 1) * p.ldc + p.N);
  const bool sc1 = sc1_ok(plane);
  const __amdgpu_buffer_rsrc_t rs = sc1_rsrc(dst, sc1 ? plane : 0);
  const float* bias = (!to_ws && p.bias) ? p.bias + bz * p.sBias : nullptr;
  constexpr int HR = WM / 2;             // rows per wave
  constexpr int NQ = HR * CPR / 64;      // 16-byte chunks per lane
  static_assert(NQ * 64 == HR * CPR, "chunks per lane");
  float4_t own[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = lane + 64 * i, r = grp * HR + q / CPR, c = (q % CPR) * 4;
    const int m = mw + r, n = nw + c;
    float4_t v = *reinterpret_cast<const float4_t*>(s0 + r * PF + c) + *reinterpret_cast<const float4_t*>(s1 + r * PF + c);
    own[i] = v;
    if (m >= p.M || n >= p.N) continue;
    if (bias)
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += bias[n + e];
    if (sc1) store_sc1(rs, ((long)m * ld + n) * 4, v);
    else __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(dst + (long)m * ld + n));
  }
  if constexpr (EPI == EPI_F32)
    if (p.pair) pair_finish<NQ, HR, CPR>(p, own, mw + grp * HR, nw, sp, bz, (tile * NWG + w4) * 2 + grp, lane);
}

// KG K-groups of NWG waves each (64*NWG*KG threads): group g consumes
// K-steps g, g+KG, g+2KG, ... through its own S/KG stages of the ring, so
// KG=2 puts 8 waves on a CU for one output tile (twice the loads in flight)
// without a global split-K reduce; the groups' accumulators are summed
// through LDS at the end (group 0 + group 1, fixed order).  A group's waves
// form an (NWG/2) x 2 grid over the tile: NWG = 8 with a 256-row tile gives
// every wave the same 64x64 sub-tile as NWG = 4 with 128 rows, while the CU
// holds two waves per SIMD and each byte it loads feeds twice the MFMAs
// along M.
// BT: B is [K][N] (N contiguous, config 1's layout).  Its stage holds
// B[k][n0 .. n0+127] rows (each DMA instruction fills 4 rows x 256 bytes),
// and the MFMA B fragments come out of LDS transposed by
// ds_read_b64_tr_b16: within a 16-lane group, source lane 4a+b reads 4
// halves (n 4b..4b+3) of row a, and lane j receives element j%4 of source
// lanes 4e + j/4, e = 0..3, i.e. rows 0..3 of column j.  Two such reads give
// a lane the 8 consecutive k of its column.  Only 128x128 tiles with the f32
// epilogue take this form.
// CV: A is an implicit convolution (conv_a_src): the A chunk addresses are
// recomputed for every K-step instead of advancing by the step.
// WCOL: waves across the tile's columns.  2 (every tile but one): a group's
// waves form an (NWG/2) x 2 grid.  1: the 128x96 QKV tile, one wave per 32
// rows over all 96 columns (store_qkv_frag_blocks).
template <int BM, int BN, int S, int KG, int EPI, int NWG = 4, bool BT = false, bool CV = false, int WCOL = 2>
__global__ __launch_bounds__(64 * NWG * KG) void gemm_dma_kernel(const GemmParams p) {
  static_assert(WCOL == 2 || (WCOL == 1 && EPI == EPI_QKV_FRAG && KG == 1 && !BT && !CV),
                "one wave column: the QKV fragment epilogue on one K-group only");
  constexpr int STAGE_A = BM * BK, STAGE_B = BN * BK, STAGE = STAGE_A + STAGE_B;   // halves
  static_assert(S % KG == 0 && S / KG >= 2, "each K-group owns at least two ring stages");
  static_assert(KG == 1 || NWG == 4, "K-groups are built from 4-wave groups");
  constexpr int P = S / KG - 1;   // steps a group keeps in flight while it computes
  // The B (weight) stream of the tiles with 128 or more rows -- the 1B model's
  // block GEMMs, 8-34 MB of weights each -- is loaded non-temporal: -1.3% of
  // the 1B frame.  Smaller tiles serve GEMMs whose few MB of weights the other
  // workgroups reuse from the caches (the 39M model: +2.4% with it).  The
  // [K][N] B of config 1 streams non-temporal too: 32.1 -> 31.4 us.  (What
  // still separates that kernel from the [N][K] one is texture-data time --
  // TD busy 12.3 M against 8.8 M cycles for the same L2 requests -- not LDS
  // bank conflicts, of which it has fewer.)
  constexpr int BPOL = BM >= 128 ? 2 : 0;
  __shared__ __attribute__((aligned(1024))) half_t lds[S * STAGE];
  constexpr int WM = BM / (NWG / WCOL), WN = BN / WCOL;
  constexpr int FM = WM / 32, FN = WN / 32;
  static_assert(FM * 32 == WM && FN * 32 == WN, "wave sub-tiles of whole 32x32 products");
  constexpr int NIA = BM / (8 * NWG), NIB = BN / (8 * NWG);   // load instructions per wave per step
  constexpr int NI = NIA + NIB;
  static_assert(NIA * 8 * NWG == BM && NIB * 8 * NWG == BN, "tile rows must split into whole load instructions");
  static_assert(KG == 1 || 4 * FM * FN * 16 * 64 * 4 <= S * STAGE * 2, "LDS too small for the group combine");

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / NWG, w4 = wave % NWG;
  const int wm = w4 / WCOL, wn = w4 % WCOL;

  const int total = p.Mt * p.Nt * p.split * p.batch;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int mt = L % p.Mt; L /= p.Mt;
  const int nt = L % p.Nt; L /= p.Nt;
  const int sp = L % p.split;
  const int bz = L / p.split;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = sp * p.kps;
  const int nkg = p.kps / (BK * KG);   // steps per group (host checks divisibility)

  // per-lane sources: instruction i of wave w4 fills rows (w4*NIA + i)*8 + lane/8;
  // physical chunk lane%8 <- logical chunk (lane%8) ^ ((row >> 1) & 7)
  const half_t* asrc[NIA];
  const half_t* bsrc[NIB];
  int cyb[NIA], cxb[NIA], ckq[NIA];   // implicit conv: 2*ho-1, 2*wo-1, the lane's chunk offset in K
#pragma unroll
  for (int i = 0; i < NIA; ++i) {
    const int r = (w4 * NIA + i) * 8 + (lane >> 3);
    const int q = (lane & 7) ^ ((r >> 1) & 7);
    if (CV) {
      const int m = min(m0 + r, p.M - 1), ho = m / p.cwo, wo = m - ho * p.cwo;
      cyb[i] = 2 * ho - 1; cxb[i] = 2 * wo - 1; ckq[i] = kbeg + q * 8;
      asrc[i] = nullptr;
    } else {
      asrc[i] = p.A + bz * p.sA + (long)min(m0 + r, p.M - 1) * p.lda + kbeg + q * 8;
    }
  }
  const half_t* const cimg = p.A + bz * p.sA;
  // implicit conv: the A chunk pointers of K-step ks (offset ks*BK past kbeg)
  auto conv_step = [&](const half_t** dst, int ks) {
#pragma unroll
    for (int i = 0; i < NIA; ++i) dst[i] = conv_a_src(p, cimg, cyb[i], cxb[i], ckq[i] + ks * BK);
  };
#pragma unroll
  for (int i = 0; i < NIB; ++i) {
    if (BT) {   // instruction i: stage rows (k) 4*(w4*NIB+i) .. +3, lane -> row +lane/16, physical chunk lane%16
      const int r = (w4 * NIB + i) * 4 + (lane >> 4);
      const int q = (lane & 15) ^ bt_swz(r);
      bsrc[i] = p.B + bz * p.sB + (long)(kbeg + r) * p.ldb + n0 + q * 8;
    } else {
      const int r = (w4 * NIB + i) * 8 + (lane >> 3);
      const int q = (lane & 7) ^ ((r >> 1) & 7);
      bsrc[i] = p.B + bz * p.sB + (long)min(n0 + r, p.N - 1) * p.ldb + kbeg + q * 8;
    }
  }
  static_assert(!BT || (BN == 128 && EPI == EPI_F32), "[K][N] B: 128-wide N tiles and the f32 epilogue only");
  float16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float16_t{};
  // the bias of the lane's epilogue columns, loaded before the K loop so its
  // latency hides behind the loop (older than every DMA, it has landed by the
  // first vmcnt wait)
  // the epilogues of the tiles with two or more 32x32 products per wave run
  // the MFMA with swapped operands (accumulators = D^T; see store_staged),
  // except the QKV ones and the [K][N] B path, whose transposed B reads
  // measured slower in the other operand slot (config 1: 33.2 against
  // 32.3 us).  On the 64x64 tiles (one product per wave) the 16 bias values
  // per lane cost more than the staging writes save (39M frame 0.1870 ->
  // 0.1907 ms); the 1B model's O-projection (two per wave) gains (1B frame
  // 2.047 -> 2.036 ms).
  constexpr bool SWP = EPI != EPI_QKV && EPI != EPI_QKV_FRAG && !BT && FM * FN >= 2;
  constexpr int NBC = SWP ? 16 : 1;
  float bcol[FN][NBC];
  {
    const float* bias = (p.split == 1 && EPI != EPI_PARTIALS && p.bias) ? p.bias + bz * p.sBias : nullptr;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < NBC; ++e) {
        const int n = n0 + wn * WN + j * 32 + (SWP ? 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3) : (lane & 31));
        bcol[j][e] = (bias && n < p.N) ? bias[n] : 0.f;
      }
  }

  // group step t is global step KG*t + grp, held in ring stage (KG*t + grp) % S
#pragma unroll
  for (int t = 0; t < P; ++t)
    if (t < nkg) {
      const long bko = BT ? (long)(KG * t + grp) * BK * p.ldb : (long)(KG * t + grp) * BK;
      if (CV) {
        const half_t* acv[NIA];
        conv_step(acv, KG * t + grp);
        dma_issue<NIA, NIB, STAGE_A, BPOL>(acv, bsrc, lds + (KG * t + grp) * STAGE, w4, 0, bko);
      } else {
        dma_issue<NIA, NIB, STAGE_A, BPOL>(asrc, bsrc, lds + (KG * t + grp) * STAGE, w4, (KG * t + grp) * BK, bko);
      }
    }

  int aoff[FM], boff[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) aoff[i] = (wm * WM + i * 32 + (lane & 31)) * BK;
#pragma unroll
  for (int j = 0; j < FN; ++j) boff[j] = (wn * WN + j * 32 + (lane & 31)) * BK;
  const int rsw = (lane >> 1) & 7;   // ((row >> 1) & 7) of every fragment row this lane reads
  // [K][N] B: lane (g = lane/16, a = (lane/4)%4, b = lane%4) of a transposed
  // read of fragment j, k-half h (k = 8*(g/2) + 4h .. +3 of a 16-k slice,
  // columns 16*(g%2) .. +15 of the fragment) reads row 8*(g/2) + 4h + a of the
  // slice, halves 4b..4b+3 of the fragment's 16-column block; the row's
  // swizzle does not depend on the slice (slices are 16 rows).
  int btoff[FN][2];
  if (BT) {
    const int g = lane >> 4, a = (lane >> 2) & 3, b = lane & 3;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int row = 8 * (g >> 1) + 4 * h + a;
        const int col = wn * WN + j * 32 + 16 * (g & 1) + 4 * b;
        btoff[j][h] = row * BN + (((col >> 3) ^ bt_swz(row)) << 3) + (col & 7);
      }
  }

  for (int t = 0; t < nkg; ++t) {
    const int ahead = min(P - 1, nkg - 1 - t);   // this group's later steps already in flight
    if (P >= 4 && ahead >= 3) wait_vm_lgkm0<3 * NI>();
    else if (P >= 3 && ahead >= 2) wait_vm_lgkm0<2 * NI>();
    else if (P >= 2 && ahead >= 1) wait_vm_lgkm0<NI>();
    else wait_vm_lgkm0<0>();
    lds_barrier();
    // refill the stage this group consumed at step t-1 (every wave passed the
    // barrier).  The refill's NI load instructions are spread over the k-slices
    // below, a few ahead of each slice's MFMAs: issued back to back they would
    // hold the wave at the address unit for the whole step's worth of loads
    // before its first MFMA.
    const bool refill = t + P < nkg;
    half_t* const rst = lds + ((KG * (t + P) + grp) % S) * STAGE;
    const int rko = (KG * (t + P) + grp) * BK;
    const long rbko = BT ? (long)rko * p.ldb : (long)rko;
    const half_t* acv[NIA];
    if (CV && refill) conv_step(acv, KG * (t + P) + grp);
    const half_t* const* ra = CV ? acv : asrc;
    const int rako = CV ? 0 : rko;
    const half_t* sa = lds + ((KG * t + grp) % S) * STAGE;
    const half_t* sb = sa + STAGE_A;
    // Two-deep software pipeline over the step's k-slices, each slice's
    // fragments in registers of their own: the LDS reads of slice kk+2 are
    // issued behind the MFMAs of slice kk, so reads overlap matrix work and
    // never wait for the matrix core to release a reused source register
    // (at most 2 slices = 8 reads outstanding, within lgkmcnt's range).
    constexpr int KS = BK / 16;
    half8_t af[KS][FM], bf[KS][FN];
    auto read_slice = [&](int kk) {
      const int ch = ((kk * 2 + (lane >> 5)) ^ rsw) * 8;
#pragma unroll
      for (int i = 0; i < FM; ++i) af[kk][i] = *reinterpret_cast<const half8_t*>(sa + aoff[i] + ch);
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if (BT) {
          typedef short s16x4_t __attribute__((ext_vector_type(4)));
          typedef __attribute__((address_space(3))) s16x4_t* lds_s4_t;
          const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(sb + kk * 16 * BN + btoff[j][0]));
          const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t)(sb + kk * 16 * BN + btoff[j][1]));
          const half4_t hl = __builtin_bit_cast(half4_t, lo), hh = __builtin_bit_cast(half4_t, hi);
          bf[kk][j] = half8_t{hl[0], hl[1], hl[2], hl[3], hh[0], hh[1], hh[2], hh[3]};
        } else {
          bf[kk][j] = *reinterpret_cast<const half8_t*>(sb + boff[j] + ch);
        }
      }
    };
    read_slice(0);
    read_slice(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if (refill)
        dma_issue_range<NIA, NIB, STAGE_A, BPOL>(ra, bsrc, rst, w4, rako, rbko, kk * NI / KS, (kk + 1) * NI / KS);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = SWP ? __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[kk][j], af[kk][i], acc[i][j], 0, 0, 0)
                          : __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kk][i], bf[kk][j], acc[i][j], 0, 0, 0);
      if (kk + 2 < KS) read_slice(kk + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // f32 outputs of two K-groups: the groups' sum inside the staged epilogue
  constexpr bool KG2_STAGED =
      KG == 2 && NWG == 4 && (EPI == EPI_F32 || EPI == EPI_PARTIALS) && kg2_staging_fits(BM, BN, S);
  if constexpr (KG2_STAGED) {
    if (p.vec) {
      wait_vm_lgkm0<0>();   // every wave is past its last ring read
      lds_barrier();
      store_staged_kg2<WM, WN, FM, FN, EPI, SWP, NWG>(p, acc, reinterpret_cast<char*>(lds), grp, w4, m0 + wm * WM,
                                                      n0 + wn * WN, sp, bz, (bz * p.Mt + mt) * p.Nt + nt, lane);
      return;
    }
  }
  if (KG > 1) {   // group 1 hands its partial tile to group 0 through LDS
    float* red = reinterpret_cast<float*>(lds);
    wait_vm_lgkm0<0>();
    lds_barrier();
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) red[((w4 * FM * FN + i * FN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    }
    wait_vm_lgkm0<0>();
    lds_barrier();
    if (grp == 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += red[((w4 * FM * FN + i * FN + j) * 16 + e) * 64 + lane];
    }
    if (p.vec) {   // the staged epilogue reuses the LDS that group 0 just read
      wait_vm_lgkm0<0>();
      lds_barrier();
    }
    if (grp == 1) return;   // no barrier follows
  } else if (p.vec) {       // every wave is past its last ring read
    wait_vm_lgkm0<0>();
    lds_barrier();
  }

  if (p.vec) {
    // bytes per wave: the f32 staging is the largest, or for one wave column
    // the row-major Q/K area and the transposed V area side by side
    constexpr int REGION = WCOL == 1 ? 2 * (WM * (WN + 8) + WN * (WM + 8)) : WM * (WN + 8) * 4;
    static_assert(NWG * REGION <= S * STAGE * 2, "LDS ring too small for the staged epilogue");
    if constexpr (WCOL == 1)
      store_qkv_frag_blocks<WM, WN, FM, FN>(p, acc, bcol, reinterpret_cast<char*>(lds) + w4 * REGION, m0 + wm * WM,
                                            n0 + wn * WN, lane);
    else
      store_staged<WM, WN, FM, FN, EPI, SWP, NBC>(p, acc, bcol, reinterpret_cast<char*>(lds) + w4 * REGION,
                                                  m0 + wm * WM, n0 + wn * WN, sp, bz, lane);
    return;
  }

  if (p.split > 1 || EPI == EPI_PARTIALS) {
    float* ws = p.ws + ((long)sp * p.batch + bz) * (long)p.M * p.N;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + wm * WM + i * 32 + (SWP ? (lane & 31) : 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3));
          const int n = n0 + wn * WN + j * 32 + (SWP ? 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3) : (lane & 31));
          if (m < p.M && n < p.N) ws[(long)m * p.N + n] = acc[i][j][e];
        }
    return;
  }
  void* C = (EPI == EPI_F32 || EPI == EPI_F32_RESID || EPI == EPI_EMBED)
                ? static_cast<void*>(static_cast<float*>(p.C) + bz * p.sC)
                : static_cast<void*>(static_cast<half_t*>(p.C) + bz * p.sC);
  const float* bias = p.bias ? p.bias + bz * p.sBias : nullptr;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * WM + i * 32 + (SWP ? (lane & 31) : 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3));
        const int n = n0 + wn * WN + j * 32 + (SWP ? 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3) : (lane & 31));
        if (m < p.M && n < p.N) epi_store<EPI>(p, C, bias, m, n, acc[i][j][e]);
      }
}

// [K][N] B through registers (tile 2: 128x64, two K-groups of 4 waves, a
// 6-stage ring, 3 stages per group).  A streams into LDS by LDS-DMA as in
// gemm_dma_kernel.  B does not: each thread of a group loads a 2 (k) x 8 (n)
// block of the step's 64 x 64 B tile with two 16-byte non-temporal loads
// (8 consecutive threads cover one 128-byte k-row), issued three K-steps
// ahead into registers; one step ahead of its use it interleaves the two rows
// into 8 dwords (column n: B[k][n], B[k+1][n]) and writes them into the B
// stage in an [N][K] layout, so the MFMA B fragments are plain 16-byte LDS
// reads.  Its rows are XOR-swizzled by chunk ^ (((n >> 1) ^ (n >> 4)) & 7)
// rather than the NT kernel's (n >> 1) & 7, and the upper half-wave writes
// its columns in the order j ^ 1: both the fragment reads (16 consecutive
// rows per pass) and the dword writes (64 lanes = 8 n-octets x 8 k-pairs)
// then touch every bank at most once (a CPU replay checks both).  The transposing LDS reads of the
// direct [K][N] path spend texture-data cycles (TD busy twice that of the
// [N][K] kernel for the same L2 requests); this path does not.
// Per group step t (group step u = global step 2u + group):
//   top:   wait for A(t) and B(t+1) (everything issued before step t-1), barrier
//   then:  B(t+1) registers -> its LDS stage (read at step t-2, retired by
//          the barrier of step t-1); load B(t+3); A(t+2) spread over the
//          k-slices of step t; the MFMAs of step t.
// The buffers rotate with period 3, so the loop body is instantiated per
// buffer phase (static register indices), and the group's step count is a
// multiple of 3 (checked on the host).  The loop is branch-free -- every
// step issues its B loads and A refill, the ones past the last step with the
// step index clamped, into stages no later step reads -- so the compiler's
// own wait counts for the register loads are exact (a branch in the loop
// makes it fall back to draining every load).
template <int I, class T>
__device__ __forceinline__ T& pick3(T& a, T& b, T& c) {
  if constexpr (I == 0) return a;
  else if constexpr (I == 1) return b;
  else return c;
}

__global__ __launch_bounds__(512) void gemm_kn_rb_kernel(const GemmParams p) {
  constexpr int BM = 128, BN = 64, S = 6, KG = 2, NWG = 4;
  constexpr int STAGE_A = BM * BK, STAGE_B = BN * BK, STAGE = STAGE_A + STAGE_B;   // halves
  constexpr int WM = BM / 2, WN = BN / 2, FM = WM / 32, FN = WN / 32;
  constexpr int NIA = BM / (8 * NWG);   // A LDS-DMA instructions per wave per step
  constexpr int NBL = 2;                // B register loads per lane per step
  constexpr int KS = BK / 16;
  __shared__ __attribute__((aligned(1024))) half_t lds[S * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / NWG, w4 = wave % NWG;
  const int wm = w4 >> 1, wn = w4 & 1;
  const int total = p.Mt * p.Nt * p.split * p.batch;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int mt = L % p.Mt; L /= p.Mt;
  const int nt = L % p.Nt; L /= p.Nt;
  const int sp = L % p.split;
  const int bz = L / p.split;
  const int m0 = mt * BM, n0 = nt * BN;
  const int kbeg = sp * p.kps;
  const int nkg = p.kps / (BK * KG);

  const half_t* asrc[NIA];
#pragma unroll
  for (int i = 0; i < NIA; ++i) {
    const int r = (w4 * NIA + i) * 8 + (lane >> 3);
    const int q = (lane & 7) ^ ((r >> 1) & 7);
    asrc[i] = p.A + bz * p.sA + (long)min(m0 + r, p.M - 1) * p.lda + kbeg + q * 8;
  }
  const half_t* const bnone[1] = {nullptr};
  // B: group thread tg -> k-pair kp (rows 2kp, 2kp+1 of the step), n-octet no
  const int tg = w4 * 64 + lane, kp = tg >> 3, no = tg & 7;
  const half_t* const bsr = p.B + bz * p.sB + (long)(kbeg + 2 * kp) * p.ldb + n0 + 8 * no;
  // write j of the lane: column 8no + (j ^ x), x = upper half-wave; its LDS
  // offset (halves, in a stage's B part) and the byte selector that takes the
  // column's half of each row word (v_perm_b32: low halves 0x05040100, high 0x07060302)
  const int x = lane >> 5;
  int bw[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int n = 8 * no + (j ^ x);
    bw[j] = n * BK + ((((2 * kp) >> 3) ^ (((n >> 1) ^ (n >> 4)) & 7)) << 3) + ((2 * kp) & 7);
  }
  const unsigned bsel[2] = {x ? 0x07060302u : 0x05040100u, x ? 0x05040100u : 0x07060302u};
  float16_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = float16_t{};
  // accumulators hold D^T (operands swapped): lane's 4 consecutive e = 4 columns of one row
  constexpr int NBC = 16;
  float bcol[FN][NBC];
  {
    const float* bias = (p.split == 1 && p.bias) ? p.bias + bz * p.sBias : nullptr;
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < NBC; ++e) {
        const int n = n0 + wn * WN + j * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        bcol[j][e] = (bias && n < p.N) ? bias[n] : 0.f;
      }
  }
  // stage of group step u: (KG u + grp) % S = 2 (u % 3) + grp
  auto stage_of = [&](int u) { return lds + ((KG * u + grp) % S) * STAGE; };
  half_t* const gstage = lds + grp * STAGE;
  auto b_load = [&](u32x4_t (&r)[NBL], int u) {
    const half_t* src = bsr + (long)(KG * u + grp) * BK * p.ldb;
    r[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src));
    r[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(src + p.ldb));
  };
  auto b_store_at = [&](const u32x4_t (&r)[NBL], half_t* st) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      *reinterpret_cast<unsigned*>(st + STAGE_A + bw[j]) = __builtin_amdgcn_perm(r[1][j >> 1], r[0][j >> 1], bsel[j & 1]);
  };
  auto b_store = [&](const u32x4_t (&r)[NBL], int u) { b_store_at(r, stage_of(u)); };
  u32x4_t rb0[NBL], rb1[NBL], rb2[NBL];
  // prologue (nkg >= 3): B(0), B(1), A(0), B(2), A(1); then everything has landed and B(0) goes to LDS
  b_load(rb0, 0);
  b_load(rb1, 1);
  dma_issue<NIA, 0, STAGE_A>(asrc, bnone, stage_of(0), w4, grp * BK, 0);
  b_load(rb2, 2);
  dma_issue<NIA, 0, STAGE_A>(asrc, bnone, stage_of(1), w4, (KG + grp) * BK, 0);
  wait_vm_lgkm0<0>();
  b_store(rb0, 0);

  int aoff[FM], boff[FN];
#pragma unroll
  for (int i = 0; i < FM; ++i) aoff[i] = (wm * WM + i * 32 + (lane & 31)) * BK;
  int bsw[FN];   // the B rows' swizzle, ((n >> 1) ^ (n >> 4)) & 7
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = wn * WN + j * 32 + (lane & 31);
    boff[j] = n * BK;
    bsw[j] = ((n >> 1) ^ (n >> 4)) & 7;
  }
  const int rsw = (lane >> 1) & 7;

  // one group step; PH = t % 3: B(t+1) is in buffer (PH+1)%3, B(t+3) loads into PH.
  // LAST: the final phase (steps nkg-3 .. nkg-1) loads nothing past the end:
  // step nkg-3 refills A only, nkg-2 loads nothing, nkg-1 neither loads nor
  // stores B, so nothing is in flight when the loop ends.
  auto step = [&](auto ph, auto last, int t) {
    constexpr int PH = decltype(ph)::value;
    constexpr bool LAST = decltype(last)::value;
    auto& rs = pick3<(PH + 1) % 3>(rb0, rb1, rb2);
    auto& rl = pick3<PH>(rb0, rb1, rb2);
    // everything but the previous step's loads has landed: A(t), B(t+1)
    constexpr int PREV = !LAST || PH == 0 ? NIA + NBL : (PH == 1 ? NIA : 0);
    wait_vm_lgkm0<PREV>();
    lds_barrier();
    half_t* const st1 = gstage + 2 * ((PH + 1) % 3) * STAGE;   // stage of step t + 1
    if constexpr (!LAST || PH < 2) b_store_at(rs, st1);
    if constexpr (!LAST) b_load(rl, t + 3);
    half_t* const rst = gstage + 2 * ((PH + 2) % 3) * STAGE;   // stage of step t + 2
    const int rko = (KG * (t + 2) + grp) * BK;
    const half_t* sa = gstage + 2 * PH * STAGE;
    const half_t* sb = sa + STAGE_A;
    half8_t af[KS][FM], bf[KS][FN];
    auto read_slice = [&](int kk) {
      const int c = kk * 2 + (lane >> 5);
#pragma unroll
      for (int i = 0; i < FM; ++i) af[kk][i] = *reinterpret_cast<const half8_t*>(sa + aoff[i] + ((c ^ rsw) << 3));
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[kk][j] = *reinterpret_cast<const half8_t*>(sb + boff[j] + ((c ^ bsw[j]) << 3));
    };
    read_slice(0);
    read_slice(1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int kk = 0; kk < KS; ++kk) {
      if constexpr (!LAST || PH == 0)
        dma_issue_range<NIA, 0, STAGE_A>(asrc, bnone, rst, w4, rko, 0, kk * NIA / KS, (kk + 1) * NIA / KS);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(bf[kk][j], af[kk][i], acc[i][j], 0, 0, 0);
      if (kk + 2 < KS) read_slice(kk + 2);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using P0 = std::integral_constant<int, 0>;
  using P1 = std::integral_constant<int, 1>;
  using P2 = std::integral_constant<int, 2>;
  using Mid = std::false_type;
  using Last = std::true_type;
  for (int t = 0; t + 3 < nkg; t += 3) {
    step(P0{}, Mid{}, t);
    step(P1{}, Mid{}, t + 1);
    step(P2{}, Mid{}, t + 2);
  }
  step(P0{}, Last{}, nkg - 3);
  step(P1{}, Last{}, nkg - 2);
  step(P2{}, Last{}, nkg - 1);

  if (p.vec) {   // the two groups' sum inside the staged epilogue
    static_assert(2 * NWG * WM * (WN + 8) * 4 <= S * STAGE * 2, "LDS ring too small for the staged epilogue");
    wait_vm_lgkm0<0>();
    lds_barrier();
    store_staged_kg2<WM, WN, FM, FN, EPI_F32, true, NWG>(p, acc, reinterpret_cast<char*>(lds), grp, w4, m0 + wm * WM,
                                                         n0 + wn * WN, sp, bz, (bz * p.Mt + mt) * p.Nt + nt, lane);
    return;
  }
  // group 1 hands its partial tile to group 0 through LDS
  {
    float* red = reinterpret_cast<float*>(lds);
    wait_vm_lgkm0<0>();
    lds_barrier();
    if (grp == 1) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) red[((w4 * FM * FN + i * FN + j) * 16 + e) * 64 + lane] = acc[i][j][e];
    }
    wait_vm_lgkm0<0>();
    lds_barrier();
    if (grp == 0) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][j][e] += red[((w4 * FM * FN + i * FN + j) * 16 + e) * 64 + lane];
    }
    if (grp == 1) return;
  }
  float* const out = p.split > 1 ? p.ws + ((long)sp * p.batch + bz) * (long)p.M * p.N
                                 : static_cast<float*>(p.C) + bz * p.sC;
  const long ld = p.split > 1 ? p.N : p.ldc;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + wm * WM + i * 32 + (lane & 31);
        const int n = n0 + wn * WN + j * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (m < p.M && n < p.N) out[(long)m * ld + n] = acc[i][j][e] + bcol[j][e];
      }
}

// B given as [K][N] (N contiguous, config 1's layout) is turned into the
// [N][K] layout the LDS-DMA kernel streams: 64x64 tiles through LDS, 16-byte
// global reads and writes.  The LDS pitch of 66 halves (33 words) keeps the
// column reads of the write-out on distinct banks.
__global__ __launch_bounds__(256) void transpose_kn_kernel(const half_t* __restrict__ src, long ld_src, long s_src,
                                                           half_t* __restrict__ dst, long s_dst, int K, int N) {
  __shared__ half_t t[64][66];
  const int k0 = blockIdx.x * 64, n0 = blockIdx.y * 64;
  src += blockIdx.z * s_src;
  dst += blockIdx.z * s_dst;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = tid / 8 + 32 * i, c = (tid % 8) * 8;   // k row r, n columns c..c+7
    if (n0 + c < N) {
      const half8_t v = *reinterpret_cast<const half8_t*>(src + (long)(k0 + r) * ld_src + n0 + c);
#pragma unroll
      for (int e = 0; e < 8; ++e) t[r][c + e] = v[e];
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int r = tid / 8 + 32 * i, c = (tid % 8) * 8;   // n row r, k columns c..c+7
    if (n0 + r < N) {
      half8_t v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = t[c + e][r];
      *reinterpret_cast<half8_t*>(dst + (long)(n0 + r) * K + k0 + c) = v;
    }
  }
}

// LDS-DMA kernel configurations: KG = 2 (8 waves) where K allows, else KG = 1.
template <int BM, int BN, int EPI>
void launch_dma_tile(const GemmParams& p, bool kg2, hipStream_t s) {
  const int grid = p.Mt * p.Nt * p.split * p.batch;
  constexpr int stage_bytes = (BM + BN) * BK * 2;
  constexpr int S1 = (5 * stage_bytes <= 163840) ? 5 : 4;
  constexpr int S2 = dma_stages_kg2(BM, BN);
  if (kg2) CK_LAUNCH((gemm_dma_kernel<BM, BN, S2, 2, EPI>), dim3(grid), dim3(512), 0, s, p);
  else CK_LAUNCH((gemm_dma_kernel<BM, BN, S1, 1, EPI>), dim3(grid), dim3(256), 0, s, p);
  CK_LAUNCHED("gemm_dma");
}

// LDS-DMA tiles with an implicit-convolution A (tile codes 1-8).
template <int BM, int BN, int EPI>
void launch_dma_tile_cv(const GemmParams& p, bool kg2, hipStream_t s) {
  const int grid = p.Mt * p.Nt * p.split * p.batch;
  constexpr int stage_bytes = (BM + BN) * BK * 2;
  constexpr int S1 = (5 * stage_bytes <= 163840) ? 5 : 4;
  constexpr int S2 = dma_stages_kg2(BM, BN);
  if (kg2) CK_LAUNCH((gemm_dma_kernel<BM, BN, S2, 2, EPI, 4, false, true>), dim3(grid), dim3(512), 0, s, p);
  else CK_LAUNCH((gemm_dma_kernel<BM, BN, S1, 1, EPI, 4, false, true>), dim3(grid), dim3(256), 0, s, p);
  CK_LAUNCHED("gemm_dma_conv");
}

template <int EPI>
void launch_epi_cv(int tile, const GemmParams& p, hipStream_t s) {
  if (tile == 15) {   // 32x64, two waves (short M: the conv stem's later layers)
    CK_LAUNCH((gemm_dma_kernel<32, 64, 5, 1, EPI, 2, false, true>), dim3(p.Mt * p.Nt * p.split * p.batch), dim3(128),
              0, s, p);
    CK_LAUNCHED("gemm_dma_conv");
    return;
  }
  const int c = tile % 10;
  const bool kg2 = c <= 4 && p.kps % (2 * BK) == 0;
  switch (c > 4 ? c - 4 : c) {
    case 1: launch_dma_tile_cv<128, 128, EPI>(p, kg2, s); break;
    case 2: launch_dma_tile_cv<128, 64, EPI>(p, kg2, s); break;
    case 3: launch_dma_tile_cv<64, 128, EPI>(p, kg2, s); break;
    default: launch_dma_tile_cv<64, 64, EPI>(p, kg2, s); break;
  }
}

// LDS-DMA tiles for a [K][N] B (f32 output): 128x128 with two K-groups (tile
// 1) or one, and 256x128 with 8 waves in one K-group (tile 9, 3-stage ring).
void launch_dma_bt(const GemmParams& p, int tile, bool kg2, hipStream_t s) {
  const int grid = p.Mt * p.Nt * p.split * p.batch;
  if (tile == 9) CK_LAUNCH((gemm_dma_kernel<256, 128, 3, 1, EPI_F32, 8, true>), dim3(grid), dim3(512), 0, s, p);
  else if (tile == 2) CK_LAUNCH(gemm_kn_rb_kernel, dim3(grid), dim3(512), 0, s, p);
  else if (kg2) CK_LAUNCH((gemm_dma_kernel<128, 128, 4, 2, EPI_F32, 4, true>), dim3(grid), dim3(512), 0, s, p);
  else CK_LAUNCH((gemm_dma_kernel<128, 128, 5, 1, EPI_F32, 4, true>), dim3(grid), dim3(256), 0, s, p);
  CK_LAUNCHED("gemm_dma_bt");
}

// 256x128 tile: 8 waves of 64x64, one K-group, 3-stage ring (3 x 48 KB).
template <int EPI>
void launch_dma_tile8(const GemmParams& p, hipStream_t s) {
  const int grid = p.Mt * p.Nt * p.split * p.batch;
  CK_LAUNCH((gemm_dma_kernel<256, 128, 3, 1, EPI, 8>), dim3(grid), dim3(512), 0, s, p);
  CK_LAUNCHED("gemm_dma");
}

template <int BM, int BN, bool BKN, int EPI>
void launch_tile(const GemmParams& p, hipStream_t s) {
  const int grid = p.Mt * p.Nt * p.split * p.batch;
  CK_LAUNCH((gemm_kernel<BM, BN, BKN, EPI>), dim3(grid), dim3(256), 0, s, p);
  CK_LAUNCHED("gemm");
}

// tile codes (BM x BN): 1 128x128, 2 128x64, 3 64x128, 4 64x64.
//   1-4: LDS-DMA kernel with two K-groups (8 waves) when K per split is a
//        multiple of 128, else one group;  5-8: LDS-DMA, one group (a [K][N]
//        B is first transposed into the workspace);
//   9: 256x128 on the LDS-DMA kernel with 8 waves in one K-group;
//   10: 128x96, one wave column (the QKV fragment epilogue only);
//   11-14: register-staged kernel (a [K][N] B is transposed in registers);
//   15: 32x64 on the LDS-DMA kernel with two waves ([N][K] B; implicit conv too).
template <bool BKN, int EPI>
void launch_epi(int tile, const GemmParams& p, hipStream_t s) {
  const int c = tile % 10;
  if (tile == 10) {   // 128x96, one wave column, 5-stage ring (5 x 28 KB): the QKV fragment epilogue only
    if constexpr (!BKN && EPI == EPI_QKV_FRAG) {
      CK_LAUNCH((gemm_dma_kernel<128, 96, 5, 1, EPI, 4, false, false, 1>), dim3(p.Mt * p.Nt), dim3(256), 0, s, p);
      CK_LAUNCHED("gemm_dma");
      return;
    }
    throw Error("gemm: tile 10 (128x96) serves the QKV fragment epilogue only");
  }
  if (tile == 15) {   // 32x64, two waves of 32x32, 5-stage ring (5 x 12 KB): more workgroups for short M
    if constexpr (!BKN) {
      CK_LAUNCH((gemm_dma_kernel<32, 64, 5, 1, EPI, 2>), dim3(p.Mt * p.Nt * p.split * p.batch), dim3(128), 0, s, p);
      CK_LAUNCHED("gemm_dma");
      return;
    }
    throw Error("gemm: tile 15 (32x64) takes B as [N][K] only");
  }
  if (!BKN && tile == 9) {
    launch_dma_tile8<EPI>(p, s);
    return;
  }
  if (!BKN && tile < 10) {
    const bool kg2 = c <= 4 && p.kps % (2 * BK) == 0;
    switch (c > 4 ? c - 4 : c) {
      case 1: launch_dma_tile<128, 128, EPI>(p, kg2, s); break;
      case 2: launch_dma_tile<128, 64, EPI>(p, kg2, s); break;
      case 3: launch_dma_tile<64, 128, EPI>(p, kg2, s); break;
      default: launch_dma_tile<64, 64, EPI>(p, kg2, s); break;
    }
    return;
  }
  switch (c) {
    case 1: launch_tile<128, 128, BKN, EPI>(p, s); break;
    case 2: launch_tile<128, 64, BKN, EPI>(p, s); break;
    case 3: launch_tile<64, 128, BKN, EPI>(p, s); break;
    default: launch_tile<64, 64, BKN, EPI>(p, s); break;
  }
}

template <int EPI, int NSTEP>
void launch_reduce_gemv(const GemmParams& p, int nr, GemvArgs g, bool nt, hipStream_t s) {
  g.rows_per_wg = gemv_rows_per_wg(g.rows, 0);
  const int nb = ceil_div(g.rows, g.rows_per_wg);
  if (nt) CK_LAUNCH((splitk_reduce_gemv_kernel<EPI, NSTEP, true>), dim3(nr + nb), dim3(256), 0, s, p, nr, g, nb);
  else CK_LAUNCH((splitk_reduce_gemv_kernel<EPI, NSTEP, false>), dim3(nr + nb), dim3(256), 0, s, p, nr, g, nb);
}

// The split-K reduce, with the GEMV of `rider` (rows > 0) riding along.
template <int EPI>
void launch_reduce(const GemmParams& p, hipStream_t s, const GemvRider* rider = nullptr) {
  const long n = (long)p.M * p.N * p.batch / ((p.N & 3) == 0 ? 4 : 1);
  CK_REQUIRE((reinterpret_cast<uintptr_t>(p.ws) & 15) == 0, "gemm: split-K workspace must be 16-byte aligned");
  const int nr = (int)((n + 255) / 256);
  if (!rider || rider->rows <= 0) {
    CK_LAUNCH(splitk_reduce_kernel<EPI>, dim3(nr), dim3(256), 0, s, p);
    CK_LAUNCHED("splitk_reduce");
    return;
  }
  const GemvRider& r = *rider;
  CK_REQUIRE(r.W && r.x && r.y && r.K > 0 && r.K % 8 == 0 && r.K <= 8 * GEMV_STEP_COLS,
             "gemm: rider GEMV needs W, x, y and K a multiple of 8 up to 16384");
  CK_REQUIRE(((reinterpret_cast<uintptr_t>(r.W) | reinterpret_cast<uintptr_t>(r.x)) & 15) == 0,
             "gemm: rider GEMV W and x must be 16-byte aligned");
  GemvArgs g{};
  g.W = r.W; g.x = r.x; g.bias = r.bias; g.y = r.y;
  g.rows = r.rows; g.K = r.K; g.ldw = r.K; g.act = GEMV_NONE;
  switch (ceil_div(r.K, GEMV_STEP_COLS)) {
    case 1: launch_reduce_gemv<EPI, 1>(p, nr, g, r.stream, s); break;
    case 2: launch_reduce_gemv<EPI, 2>(p, nr, g, r.stream, s); break;
    case 3: launch_reduce_gemv<EPI, 3>(p, nr, g, r.stream, s); break;
    case 4: launch_reduce_gemv<EPI, 4>(p, nr, g, r.stream, s); break;
    case 5: launch_reduce_gemv<EPI, 5>(p, nr, g, r.stream, s); break;
    case 6: launch_reduce_gemv<EPI, 6>(p, nr, g, r.stream, s); break;
    case 7: launch_reduce_gemv<EPI, 7>(p, nr, g, r.stream, s); break;
    default: launch_reduce_gemv<EPI, 8>(p, nr, g, r.stream, s); break;
  }
  CK_LAUNCHED("splitk_reduce_gemv");
}

// A [K][N] B on the two-K-group 128x128 LDS-DMA tile is streamed into LDS as
// it lies and read transposed (no transpose pass, no workspace for it).
// (A and B are required to be 16-byte aligned for every launch.)
bool bt_direct(const GemmDesc& d) {
  if (!d.b_kn) return false;
  if (d.tile == 2)   // B through registers: whole 3-step phases of two K-groups
    return d.N % 64 == 0 && (d.K / d.split) % (6 * BK) == 0;
  if (d.N % 128 != 0) return false;
  if (d.tile == 1) return (d.K / d.split) % (2 * BK) == 0;
  return d.tile == 9;   // 256x128, 8 waves in one K-group
}

// Ticket counters of the in-kernel split-2 finish (pair_finish): a static
// per-device array, zero when the code object loads; every launch leaves the
// counters it uses even.  Each stream gets a slot of its own on first use,
// so split-2 GEMMs running at the same time on different streams never share
// a counter; once every slot is taken, further streams get the reduce
// launch.  A captured graph keeps the slot of the stream it was captured on:
// replaying it on another stream while the capturing stream runs split-2
// GEMMs races on that slot.
constexpr int kPairSlots = 16;
constexpr int kPairTickets = 8192;   // counters per slot
constexpr int kPairDevices = 64;
__device__ __align__(256) unsigned pair_tickets[kPairSlots * kPairTickets];

std::mutex g_pair_mu;
unsigned* g_pair_base[kPairDevices] = {};
std::vector<std::pair<int, hipStream_t>> g_pair_slots;   // (device, stream), in order of first use

// The ticket slot for a launch on stream s of the current device, or null
// (no slot left, or the stream belongs to another device).
unsigned* pair_slot(hipStream_t s) {
  int dev = -1;
  CK_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= kPairDevices) return nullptr;
  if (s) {
    hipDevice_t sdev = -1;
    CK_HIP(hipStreamGetDevice(s, &sdev));
    if (sdev != dev) return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_pair_mu);
  if (!g_pair_base[dev]) {
    void* q = nullptr;
    CK_HIP(hipGetSymbolAddress(&q, HIP_SYMBOL(pair_tickets)));
    CK_REQUIRE(q != nullptr, "gemm: split-K ticket array has no device address");
    g_pair_base[dev] = static_cast<unsigned*>(q);
  }
  int slot = -1, used = 0;
  for (const auto& e : g_pair_slots) {
    if (e.first != dev) continue;
    if (e.second == s) slot = used;
    ++used;
  }
  if (slot < 0) {
    if (used >= kPairSlots) return nullptr;
    g_pair_slots.emplace_back(dev, s);
    slot = used;
  }
  return g_pair_base[dev] + (size_t)slot * kPairTickets;
}

int tile_base(int tile) { const int c = tile % 10; return c > 4 ? c - 4 : c; }
bool tile_dma(int tile) { return tile <= 10 || tile == 15; }
int tile_bm(int tile) {
  return tile == 9 ? 256 : tile == 10 ? 128 : tile == 15 ? 32 : (tile_base(tile) == 1 || tile_base(tile) == 2) ? 128 : 64;
}
int tile_bn(int tile) {
  return tile == 9 ? 128 : tile == 10 ? 96 : tile == 15 ? 64 : (tile_base(tile) == 1 || tile_base(tile) == 3) ? 128 : 64;
}

}  // namespace

size_t gemm_plan(GemmDesc& d) {
  CK_REQUIRE(d.M > 0 && d.N > 0 && d.K > 0 && d.batch > 0, "gemm: empty problem");
  CK_REQUIRE(d.K % BK == 0, "gemm: K must be a multiple of 64 (pad K)");
  if (d.tile == 0 && d.b_kn && d.split == 0 && d.N % 64 == 0) {
    // A [K][N] B with enough 128x64 tiles to fill the GPU at a split whose K
    // per split makes whole 3-step phases of the register-staged kernel:
    // that kernel (config 1: 30.0-31.3 us at split 2, against 31.2-32.6 us
    // for the 128x128 transposing-read tile at split 4).
    const long t2 = (long)ceil_div(d.M, 128) * (d.N / 64) * d.batch;
    int s2 = 0;
    for (int c = 1; c <= 8; ++c)
      if (t2 * c <= 256 && d.K % (c * 6 * BK) == 0) s2 = c;
    if (t2 >= 64 && s2 > 0) {
      d.tile = 2;
      d.split = s2;
    }
  }
  if (d.tile == 0) {
    // 128-wide tiles unless a dimension is small; 64x64 when 128-wide tiles
    // leave most of the 256 CUs without a tile.
    int bm = d.M <= 64 ? 64 : 128, bn = d.N <= 64 ? 64 : 128;
    const long t = (long)ceil_div(d.M, bm) * ceil_div(d.N, bn) * d.batch;
    if (t < 64) bm = bn = 64;
    d.tile = bm == 128 ? (bn == 128 ? 1 : 2) : (bn == 128 ? 3 : 4);
  }
  CK_REQUIRE((d.tile >= 1 && d.tile <= 15), "gemm: unknown tile code");
  CK_REQUIRE(d.tile != 15 || !d.b_kn, "gemm: tile 15 (32x64) takes B as [N][K]");
  CK_REQUIRE(d.tile != 10 || (d.epi == EPI_QKV_FRAG && !d.b_kn && d.conv_c == 0),
             "gemm: tile 10 (128x96) serves the QKV fragment epilogue only");
  if (d.b_kn && !tile_dma(d.tile))
    CK_REQUIRE(d.tile == 11 || d.tile == 13, "gemm: [K][N] B on the register-staged kernel needs a 128-wide N tile");
  const long tiles = (long)ceil_div(d.M, tile_bm(d.tile)) * ceil_div(d.N, tile_bn(d.tile)) * d.batch;
  if (d.split == 0) {
    // K of 16 steps or more: the largest split (<= 16) that divides the
    // K-steps, leaves each split at least two of them and keeps the grid
    // within one wave of 256 CUs.  Shorter K is not split: the partials and
    // the reduce launch cost more than the extra workgroups gain (measured
    // on the conv stem: K = 576 runs 8.4 us unsplit, 10.0 us split in 3).
    const int ksteps = d.K / BK;
    int s = 1;
    if (ksteps >= 16)
      for (int c = 2; c <= 16; ++c)
        if (ksteps % c == 0 && ksteps / c >= 2 && tiles * c <= 256) s = c;
    d.split = s;
  }
  CK_REQUIRE(d.split >= 1 && d.K % (BK * d.split) == 0, "gemm: K must split into multiples of 64");
  // workspace: split-K partials, then (a [K][N] B on the LDS-DMA kernel) B transposed to [N][K] f16
  const size_t partials = (d.split > 1 || d.epi == EPI_PARTIALS) ? (size_t)d.split * d.batch * d.M * d.N : 0;
  const size_t bt = (d.b_kn && tile_dma(d.tile) && !bt_direct(d)) ? ((size_t)d.batch * d.N * d.K + 1) / 2 : 0;
  return partials + bt;
}

void launch_gemm(GemmDesc d, hipStream_t s) {
  const size_t need = gemm_plan(d);
  CK_REQUIRE(d.A && d.B && (d.C || d.epi == EPI_PARTIALS), "gemm: null operand");
  const bool conv = d.conv_c > 0;
  if (conv) {
    const int Ho = (d.conv_h - 1) / 2 + 1, Wo = (d.conv_w - 1) / 2 + 1;
    CK_REQUIRE(d.conv_c >= 8 && (d.conv_c & (d.conv_c - 1)) == 0 && d.conv_h > 0 && d.conv_w > 0,
               "gemm: implicit conv needs a power-of-two channel count >= 8");
    CK_REQUIRE(d.M == Ho * Wo && d.K == ((9 * d.conv_c + BK - 1) / BK) * BK,
               "gemm: implicit conv needs M = output pixels, K = 9C rounded up to 64");
    CK_REQUIRE(d.sA >= (long)d.conv_h * d.conv_w * d.conv_c || d.batch == 1, "gemm: implicit conv batch stride");
    CK_REQUIRE(d.zero16 && (reinterpret_cast<uintptr_t>(d.zero16) & 15) == 0,
               "gemm: implicit conv needs 16 zero bytes (16-byte aligned)");
    CK_REQUIRE(!d.b_kn && tile_dma(d.tile) && d.tile != 9 && d.epi == EPI_F16_BIAS_RELU,
               "gemm: implicit conv runs on the LDS-DMA tiles 1-8 and 15 with the bias+ReLU epilogue");
  } else {
    CK_REQUIRE(d.lda >= d.K && d.lda % 8 == 0, "gemm: lda must be >= K and a multiple of 8");
  }
  if (d.b_kn) {
    CK_REQUIRE(d.ldb >= d.N && d.ldb % 8 == 0 && d.N % 8 == 0, "gemm: [K][N] B needs N, ldb multiples of 8");
    CK_REQUIRE(d.epi == EPI_F32, "gemm: [K][N] B supports the f32 epilogue only");
  } else {
    CK_REQUIRE(d.ldb >= d.K && d.ldb % 8 == 0, "gemm: ldb must be >= K and a multiple of 8");
  }
  // QKV: only the first qk_cols columns are stored row-major in C
  if (d.epi != EPI_PARTIALS)
    CK_REQUIRE(d.ldc >= (d.c_nm ? d.M : (d.epi == EPI_QKV || d.epi == EPI_QKV_FRAG) ? d.qk_cols : d.N),
               "gemm: ldc must be >= N (>= qk_cols for QKV, >= M for a transposed store)");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(d.A) & 15) == 0 && (reinterpret_cast<uintptr_t>(d.B) & 15) == 0,
             "gemm: A and B must be 16-byte aligned");
  CK_REQUIRE(d.sA % 8 == 0 && d.sB % 8 == 0, "gemm: batch strides must keep 16-byte alignment");
  if (d.epi == EPI_QKV || d.epi == EPI_QKV_FRAG)
    CK_REQUIRE(d.vt && d.qk_cols > 0 && d.qk_cols < d.N && d.vt_ld >= d.M, "gemm: bad QKV split");
  if (need) CK_REQUIRE(d.ws && d.ws_floats >= need, "gemm: split-K workspace missing or too small");
  CK_REQUIRE(conv || (long)d.M * d.lda < (1L << 31) * 8, "gemm: A too large");

  GemmParams p;
  p.A = d.A; p.B = d.B; p.C = d.C; p.bias = d.bias; p.ws = d.ws; p.vt = d.vt;
  p.lda = d.lda; p.ldb = d.ldb; p.ldc = d.ldc; p.vt_ld = d.vt_ld;
  p.sA = d.sA; p.sB = d.sB; p.sC = d.sC; p.sBias = d.sBias;
  p.M = d.M; p.N = d.N; p.K = d.K; p.split = d.split; p.kps = d.K / d.split; p.batch = d.batch;
  p.Mt = ceil_div(d.M, tile_bm(d.tile)); p.Nt = ceil_div(d.N, tile_bn(d.tile));
  p.qk_cols = d.qk_cols;
  p.head_dim = d.head_dim;
  p.pos = d.pos;
  p.ctx = d.ctx;
  p.cc_log2 = conv ? __builtin_ctz(d.conv_c) : 0;
  p.ch = d.conv_h; p.cw = d.conv_w; p.cwo = conv ? (d.conv_w - 1) / 2 + 1 : 0;
  p.zero = d.zero16;
  CK_REQUIRE(!d.c_nm || (d.split > 1 && d.epi == EPI_F16_BIAS_RELU && (d.tile <= 8 || d.tile == 15)),
             "gemm: a transposed C store is done by the split-K reduce of the bias+ReLU epilogue only");
  p.c_nm = d.c_nm;
  if (d.epi == EPI_EMBED)
    CK_REQUIRE(d.pos && d.ctx && (reinterpret_cast<uintptr_t>(d.pos) & 7) == 0 &&
                   (reinterpret_cast<uintptr_t>(d.ctx) & 15) == 0,
               "gemm: the embedding epilogue needs pos (8-byte aligned) and ctx (16-byte aligned)");
  {
    // the staged epilogue writes 16-byte chunks: 8 halves / 4 floats per chunk
    const auto al16 = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
    bool v = !(d.b_kn && !tile_dma(d.tile)) && d.N % 8 == 0;
    if (d.split > 1 || d.epi == EPI_PARTIALS) {
      v = v && al16(d.ws);
    } else {
      const int el = (d.epi == EPI_F32 || d.epi == EPI_F32_RESID || d.epi == EPI_EMBED) ? 4 : 8;
      v = v && al16(d.C) && d.ldc % el == 0 && d.sC % el == 0;
      // (the 128x96 tile's epilogue takes the Q/K/V boundary per 32-column block)
      if (d.epi == EPI_QKV || d.epi == EPI_QKV_FRAG)
        v = v && d.qk_cols % (d.tile == 10 ? 32 : tile_bn(d.tile)) == 0 && d.M % 8 == 0 && d.vt_ld % 8 == 0 &&
            al16(d.vt);
    }
    p.vec = v ? 1 : 0;
  }
  // Split 2 with an f32 output on a kernel with the two-group staged
  // epilogue (the [K][N] register-B tile 2; [N][K] LDS-DMA tiles 1-4 with
  // two K-groups whose staging fits the ring) finishes in the kernel
  // (pair_finish) instead of a reduce launch.  Its partial planes must be
  // addressable by 32-bit buffer offsets (device-scope stores and loads).
  p.pair = nullptr;
  {
    const int bm = tile_bm(d.tile), bn = tile_bn(d.tile);
    const bool staged = d.b_kn ? (d.tile == 2 && bt_direct(d))
                               : (d.tile >= 1 && d.tile <= 4 && p.kps % (2 * BK) == 0 &&
                                  kg2_staging_fits(bm, bn, dma_stages_kg2(bm, bn)));
    const long tickets = (long)d.batch * p.Mt * p.Nt * 4 * 2;
    if (staged && d.split == 2 && d.epi == EPI_F32 && p.vec && !conv && 4L * d.M * d.N < (1L << 31) &&
        tickets <= kPairTickets)
      p.pair = pair_slot(s);
  }
  if (d.epi == EPI_QKV_FRAG) {
    const int dh = d.qk_cols / 2;
    // columns a wave's epilogue keeps within one head: its sub-tile's, or on
    // the 128x96 tile each 32-column block's
    const int wn = d.tile == 10 ? 32 : tile_bn(d.tile) / 2;
    CK_REQUIRE(d.head_dim >= wn && (d.head_dim & (d.head_dim - 1)) == 0 && d.qk_cols % 2 == 0 &&
                   dh % d.head_dim == 0 && d.N == 3 * dh && d.M % 32 == 0 && d.N % tile_bn(d.tile) == 0,
               "gemm: QKV fragment epilogue needs N = 3d, d % head_dim == 0, head_dim a power of two no smaller "
               "than a wave's columns, M % 32 == 0");
    CK_REQUIRE(d.split == 1 && d.batch == 1 && tile_dma(d.tile) && p.vec,
               "gemm: QKV fragment epilogue needs split 1, batch 1, an LDS-DMA tile and aligned outputs");
    // Q/K and V fragments leave through raw buffer stores addressed by 32-bit offsets
    CK_REQUIRE(2L * d.M * d.qk_cols < (1L << 31) && 2L * d.M * (d.N - d.qk_cols) < (1L << 31),
               "gemm: QKV fragment outputs must be under 2 GiB each");
  }
  CK_REQUIRE(d.rider.rows <= 0 || (conv && d.split > 1),
             "gemm: a rider GEMV goes with the split-K reduce of an implicit conv");
  if (conv) {
    launch_epi_cv<EPI_F16_BIAS_RELU>(d.tile, p, s);
    if (d.split > 1) launch_reduce<EPI_F16_BIAS_RELU>(p, s, &d.rider);
    return;
  }
  if (d.b_kn && !tile_dma(d.tile)) {
    launch_epi<true, EPI_F32>(d.tile, p, s);
    if (d.split > 1) launch_reduce<EPI_F32>(p, s);
    return;
  }
  if (bt_direct(d)) {
    // the [K][N] B straight into LDS, fragments read transposed (no transpose
    // pass).  Only with two K-groups: on one (tile 5) the doubled fragment
    // reads cost more than the transpose pass saves (config 1: 44.6 against
    // 33.2 us; two K-groups 32.6 against 34.9 us).
    launch_dma_bt(p, d.tile, true, s);
    if (d.split > 1 && !p.pair) launch_reduce<EPI_F32>(p, s);
    return;
  }
  if (d.b_kn) {   // transpose B into the workspace tail, then the NT LDS-DMA kernel
    const size_t partials = (d.split > 1) ? (size_t)d.split * d.batch * d.M * d.N : 0;
    half_t* bt = reinterpret_cast<half_t*>(d.ws + partials);
    CK_REQUIRE((reinterpret_cast<uintptr_t>(bt) & 15) == 0, "gemm: workspace must be 16-byte aligned");
    CK_LAUNCH(transpose_kn_kernel, dim3(d.K / 64, ceil_div(d.N, 64), d.batch), dim3(256), 0, s, d.B, d.ldb,
                       d.sB, bt, (long)d.N * d.K, d.K, d.N);
    CK_LAUNCHED("transpose_kn");
    p.B = bt;
    p.ldb = d.K;
    p.sB = (long)d.N * d.K;
    launch_epi<false, EPI_F32>(d.tile, p, s);
    if (d.split > 1) launch_reduce<EPI_F32>(p, s);
    return;
  }
  switch (d.epi) {
    case EPI_F32: launch_epi<false, EPI_F32>(d.tile, p, s); if (d.split > 1 && !p.pair) launch_reduce<EPI_F32>(p, s); break;
    case EPI_F16_BIAS: launch_epi<false, EPI_F16_BIAS>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_F16_BIAS>(p, s); break;
    case EPI_F16_BIAS_RELU: launch_epi<false, EPI_F16_BIAS_RELU>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_F16_BIAS_RELU>(p, s); break;
    case EPI_F16_BIAS_GELU: launch_epi<false, EPI_F16_BIAS_GELU>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_F16_BIAS_GELU>(p, s); break;
    case EPI_F32_RESID: launch_epi<false, EPI_F32_RESID>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_F32_RESID>(p, s); break;
    case EPI_EMBED: launch_epi<false, EPI_EMBED>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_EMBED>(p, s); break;
    case EPI_QKV: launch_epi<false, EPI_QKV>(d.tile, p, s); if (d.split > 1) launch_reduce<EPI_QKV>(p, s); break;
    case EPI_PARTIALS: launch_epi<false, EPI_PARTIALS>(d.tile, p, s); break;
    case EPI_QKV_FRAG: launch_epi<false, EPI_QKV_FRAG>(d.tile, p, s); break;
    default: throw Error("gemm: unknown epilogue");
  }
}

}  // namespace ck
