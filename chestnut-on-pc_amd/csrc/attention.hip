// Non-causal multi-head attention for the token block of the driving model.
//
// The reference's attention lives in comma's pickle as WMMA GEMM kernels
// (NOTES.md:84-104); this is the gfx950 form of the same f16-input,
// f32-accumulate products with an f32 softmax between them.
//
// One workgroup = 32 queries of one head (T=512, 16 heads: 256 workgroups,
// one per CU), split over the keys: wave w owns keys [w*KPW, (w+1)*KPW) for
// all 32 queries and needs nothing from the other waves until the end:
//   1. S^T = K Q^T * scale*log2(e) for its keys with v_mfma_f32_16x16x32_f16
//      (A = 16 keys x 32 head dims of K, B = Q^T); lane (g = l/16, r = l%16)
//      holds keys 4g..4g+3 of every 16-key tile for query r;
//   2. a wave-local softmax numerator: per query the max m_w over the wave's
//      keys (lane-local, then xor-16/xor-32 exchanges), e = 2^(s - m_w) on
//      the hardware exp2, l_w = sum of e; e is rounded to f16 (values in
//      (0, 1]) and is, as it stands in the registers, the A operand of P.V:
//      the two 16-key tiles of a 32-key block give lane (g, r) the keys
//      {4g..4g+3, 16+4g..16+4g+3} of query r;
//   3. O_w = e . V over the wave's keys, B = V in the same permuted key order
//      (the QKV GEMM's fragment epilogue writes V that way);
//   4. each wave leaves O_w, m_w and l_w in LDS; after one barrier the
//      threads combine 4 features of one query at a time over the waves in
//      fixed order: M = max m_w, O = sum 2^(m_w - M) O_w / sum 2^(m_w - M) l_w
//      (with the O-projection: f16 P_w = O_w / l_w, weighted by 2^(m_w - M) l_w).
// The result is deterministic; each wave streams only its own K and V.
// Workgroups are regrouped by XCD (consecutive ids land on different XCDs):
// each XCD's L2 then serves the K/V of T*hd*2*2 bytes for 2 heads.
// MFMA 16x16x32 layout (lane l): A row l%16, k = 8*(l/16)..+7; B column
// l%16, same k; D element i of lane l is row 4*(l/16)+i, column l%16.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr int ATT_TMAX = 512;
constexpr int ATT_QB = 32;   // queries per workgroup

__device__ __forceinline__ float xor_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  return fmaxf(v, __shfl_xor(v, 32));
}
__device__ __forceinline__ float xor_sum(float v) {
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}

// Waves per workgroup for T = 64*NKT keys: every wave owns 32 or 64 keys.
constexpr int att_waves(int nkt) { return nkt <= 4 ? 2 * nkt : nkt; }

// FRAG: qk / vt hold the operands in MFMA fragment order (written by the QKV
// GEMM's fragment epilogue): every fragment load of a wave is one contiguous
// KB.  Otherwise the row layouts: qk [T][2d], vt [d][T].  All of a wave's
// loads (Q, its K, its V) are issued at entry, before any MFMA.
// QT: 16-query tiles per workgroup (2: 32 queries; 1: 16, twice the
// workgroups for short sequences that would leave most CUs idle).
// OTW > 0: the output projection rides along.  The workgroup's normalised
// f16 output (QB queries x HD features of head h) goes to LDS instead of
// memory, and wave w multiplies it by columns [h*HD, (h+1)*HD) of W_o
// ([d][d], row n = output feature) for output features
// [16*OTW*w, 16*OTW*(w+1)): P_h = O_h W_o[:, h]^T, an f32 plane per head,
// opart + h*T*d, [T][d].  The planes are the split-K partials of the
// O-projection over its K = d split by heads; the next LayerNorm sums them
// in head order with the bias.  W_o's fragments are loaded at entry with
// everything else.
template <int HD, int NKT, bool FRAG, int QT = 2, int OTW = 0>
__global__ __launch_bounds__(64 * att_waves(NKT)) void attention_kernel(const half_t* __restrict__ qk,
                                                                         const half_t* __restrict__ vt,
                                                                         half_t* __restrict__ out, int n_heads,
                                                                         float scale_log2e,
                                                                         const half_t* __restrict__ wo,
                                                                         float* __restrict__ opart) {
  constexpr int QB = 16 * QT;        // queries per workgroup
  constexpr int WAVES = att_waves(NKT);
  constexpr int T = 64 * NKT;
  constexpr int KS = HD / 32;        // k-steps of the q.k products
  constexpr int KPW = T / WAVES;     // keys per wave
  constexpr int KT = KPW / 16;       // 16-key tiles per wave
  constexpr int KB = KPW / 32;       // 32-key blocks (k-steps of P.V)
  constexpr int CT = HD / 16;        // 16-wide output tiles
  static_assert(KPW % 32 == 0, "every wave must own whole 32-key blocks");
  // The waves' partial outputs: f16 P_w = O_w / l_w where the O-projection
  // rides along (half the LDS bytes of the combine: 39M frame -0.75%), f32
  // O_w otherwise (the f16 form's extra conversions cost the 1B frame +0.6%).
  // Row pitch: f32 HD + 4 floats (the 4-row scatter of each lane's
  // accumulators hits distinct banks); f16 HD + 8 halves (4 banks mod 64, so
  // the 32 lanes of a half-wave writing 8 bytes each hit 64 distinct banks).
  constexpr bool P16 = OTW > 0;
  typedef std::conditional_t<P16, half_t, float> part_t;
  constexpr int OP = P16 ? HD + 8 : HD + 4;
  __shared__ __attribute__((aligned(16))) part_t part[WAVES][QB][OP];
  __shared__ float mrow[WAVES][QB], lrow[WAVES][QB];
  constexpr int KSO = HD / 32;       // k-steps of the O-projection
  constexpr int OBP = HD + 8;        // f16 output row pitch in LDS (16-byte rows)
  __shared__ __attribute__((aligned(16))) half_t ob[OTW > 0 ? QB : 1][OBP];

  const int d = n_heads * HD;
  const int nqb = T / QB;
  const int total = nqb * n_heads;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int h = L / nqb, q0 = (L % nqb) * QB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const long ldq = 2L * d;
  const int kw0 = wave * KPW;

  // ---- all loads up front ----
  half8_t qf[QT][KS], kf[KT][KS], vb[KB][CT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[kt][ks] = *reinterpret_cast<const half8_t*>(
          FRAG ? qk + ((((long)(n_heads + h) * (T / 16) + kw0 / 16 + kt) * KS + ks) * 64 + lane) * 8
               : qk + (long)(kw0 + kt * 16 + r16) * ldq + d + h * HD + ks * 32 + g * 8);
#pragma unroll
  for (int qt = 0; qt < QT; ++qt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = *reinterpret_cast<const half8_t*>(
          FRAG ? qk + ((((long)h * (T / 16) + q0 / 16 + qt) * KS + ks) * 64 + lane) * 8
               : qk + (long)(q0 + qt * 16 + r16) * ldq + h * HD + ks * 32 + g * 8);
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      if (FRAG) {
        vb[kb][ct] = *reinterpret_cast<const half8_t*>(
            vt + ((((long)h * (HD / 16) + ct) * (T / 32) + kw0 / 32 + kb) * 64 + lane) * 8);
      } else {
        // V^T row of feature ct*16 + r16: keys 4g..4g+3 and 16+4g..16+4g+3 of the block
        const half_t* vr = vt + (long)(h * HD + ct * 16 + r16) * T + kw0 + kb * 32 + 4 * g;
        const half4_t lo = *reinterpret_cast<const half4_t*>(vr);
        const half4_t hi = *reinterpret_cast<const half4_t*>(vr + 16);
        vb[kb][ct] = half8_t{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    }
  // W_o fragments (MFMA A operand: row n = output feature, 8 k of head h's columns)
  half8_t wf[OTW > 0 ? OTW : 1][KSO];
  if constexpr (OTW > 0) {
#pragma unroll
    for (int t = 0; t < OTW; ++t)
#pragma unroll
      for (int ks = 0; ks < KSO; ++ks)
        wf[t][ks] = *reinterpret_cast<const half8_t*>(wo + (long)((wave * OTW + t) * 16 + r16) * d + h * HD +
                                                      ks * 32 + g * 8);
  }

  // ---- 1. S^T = K Q^T for this wave's keys (log2 domain) ----
  float4_t s[KT][QT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kt][ks], qf[qt][ks], a, 0, 0, 0);
      s[kt][qt] = a * scale_log2e;
    }

  // ---- 2. wave-local softmax numerator per query (column r16 of q-tile qt) ----
  half8_t pa[KB][QT];
  float lw[QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float m = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, s[kt][qt][i]);
    m = xor_max(m);
    float acc = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float e = __builtin_amdgcn_exp2f(s[2 * kb + i / 4][qt][i % 4] - m);
        acc += e;
        pa[kb][qt][i] = (half_t)e;
      }
    acc = xor_sum(acc);
    lw[qt] = acc;
    if (g == 0) {
      mrow[wave][qt * 16 + r16] = m;
      lrow[wave][qt * 16 + r16] = acc;
    }
  }

  // ---- 3. O_w = e V over this wave's keys ----
  if constexpr (P16) {
    // O_w^T = V^T e^T (operands swapped: lane (g, r16) ends with head dims
    // 16ct + 4g .. +3 of query 16qt + r16), divided by the wave's l_w: a convex
    // combination of V rows, so within V's range; one 8-byte write per tile
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const float rl = 1.0f / lw[qt];
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) a = __builtin_amdgcn_mfma_f32_16x16x32_f16(vb[kb][ct], pa[kb][qt], a, 0, 0, 0);
        *reinterpret_cast<half4_t*>(&part[wave][qt * 16 + r16][ct * 16 + 4 * g]) =
            half4_t{(half_t)(a[0] * rl), (half_t)(a[1] * rl), (half_t)(a[2] * rl), (half_t)(a[3] * rl)};
      }
    }
  } else {
    float4_t o[QT][CT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct) {
        float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) a = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[kb][qt], vb[kb][ct], a, 0, 0, 0);
        o[qt][ct] = a;
      }
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) part[wave][qt * 16 + 4 * g + i][ct * 16 + r16] = o[qt][ct][i];
  }
  __syncthreads();

  // ---- 4. combine the waves: 4 features of one query per step, in fixed wave order ----
  for (int u = threadIdx.x; u < QB * HD / 4; u += 64 * WAVES) {
    const int q = u / (HD / 4), c = (u % (HD / 4)) * 4;
    float M = mrow[0][q];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) M = fmaxf(M, mrow[w][q]);
    float den = 0.f;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < WAVES; ++w) {
      const float f = __builtin_amdgcn_exp2f(mrow[w][q] - M);
      if constexpr (P16) {
        const float fl = f * lrow[w][q];
        const half4_t pw = *reinterpret_cast<const half4_t*>(&part[w][q][c]);
        den += fl;
        acc += fl * float4_t{(float)pw[0], (float)pw[1], (float)pw[2], (float)pw[3]};
      } else {
        den += f * lrow[w][q];
        acc += f * *reinterpret_cast<const float4_t*>(&part[w][q][c]);
      }
    }
    const float rden = 1.0f / den;
    const half4_t v{(half_t)(acc[0] * rden), (half_t)(acc[1] * rden), (half_t)(acc[2] * rden), (half_t)(acc[3] * rden)};
    if constexpr (OTW > 0) {
      *reinterpret_cast<half4_t*>(&ob[q][c]) = v;
    } else {
      // device-scope cache policy for the output the O-projection reads next (-0.4% of the 1B frame)
      store_sc1(sc1_rsrc(out, 2L * T * d), ((long)(q0 + q) * d + h * HD + c) * 2, v);
    }
  }

  // ---- 5. (OTW > 0) P_h^T = W_o[n-tile, head h] O_h^T: lane (g, r16) ends with
  // output features 4g..4g+3 of the tile for query r16, one 16-byte store ----
  if constexpr (OTW > 0) {
    __syncthreads();
    half8_t of[QT][KSO];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt)
#pragma unroll
      for (int ks = 0; ks < KSO; ++ks)
        of[qt][ks] = *reinterpret_cast<const half8_t*>(&ob[qt * 16 + r16][ks * 32 + g * 8]);
    const auto pr = sc1_rsrc(opart + (long)h * T * d, 4L * T * d);
#pragma unroll
    for (int t = 0; t < OTW; ++t)
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KSO; ++ks) a = __builtin_amdgcn_mfma_f32_16x16x32_f16(wf[t][ks], of[qt][ks], a, 0, 0, 0);
        // device-scope cache policy: the LayerNorm reads the planes next
        store_sc1(pr, ((long)(q0 + qt * 16 + r16) * d + (wave * OTW + t) * 16 + 4 * g) * 4, a);
      }
  }
}

template <int HD, int NKT, bool FRAG>
void launch_t(int n_heads, const half_t* qk, const half_t* vt, half_t* out, float scale_log2e, hipStream_t s) {
  // 32 queries per workgroup, or 16 when that would leave more than half the CUs idle
  const int wg32 = (64 * NKT / ATT_QB) * n_heads;
  if (wg32 >= 128) {
    CK_LAUNCH((attention_kernel<HD, NKT, FRAG, 2>), dim3(wg32), dim3(64 * att_waves(NKT)), 0, s, qk, vt, out, n_heads,
              scale_log2e, nullptr, nullptr);
  } else {
    CK_LAUNCH((attention_kernel<HD, NKT, FRAG, 1>), dim3(2 * wg32), dim3(64 * att_waves(NKT)), 0, s, qk, vt, out,
              n_heads, scale_log2e, nullptr, nullptr);
  }
}

// With the O-projection: the same workgroup choice; OTW = d / 16 / waves
// output tiles per wave (checked by attention_oproj_tiles).
template <int HD, int NKT, int OTW>
void launch_o(int n_heads, const half_t* qk, const half_t* vt, const half_t* wo, float* opart, float scale_log2e,
              hipStream_t s) {
  const int wg32 = (64 * NKT / ATT_QB) * n_heads;
  if (wg32 >= 128) {
    CK_LAUNCH((attention_kernel<HD, NKT, true, 2, OTW>), dim3(wg32), dim3(64 * att_waves(NKT)), 0, s, qk, vt, nullptr,
              n_heads, scale_log2e, wo, opart);
  } else {
    CK_LAUNCH((attention_kernel<HD, NKT, true, 1, OTW>), dim3(2 * wg32), dim3(64 * att_waves(NKT)), 0, s, qk, vt,
              nullptr, n_heads, scale_log2e, wo, opart);
  }
}

template <int HD, int NKT>
void launch_o_t(int otw, int n_heads, const half_t* qk, const half_t* vt, const half_t* wo, float* opart,
                float scale_log2e, hipStream_t s) {
  switch (otw) {
    case 1: launch_o<HD, NKT, 1>(n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 2: launch_o<HD, NKT, 2>(n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    default: launch_o<HD, NKT, 4>(n_heads, qk, vt, wo, opart, scale_log2e, s); break;
  }
}

template <int HD>
void launch_o_hd(int T, int otw, int n_heads, const half_t* qk, const half_t* vt, const half_t* wo, float* opart,
                 float scale_log2e, hipStream_t s) {
  switch (T / 64) {
    case 1: launch_o_t<HD, 1>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 2: launch_o_t<HD, 2>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 3: launch_o_t<HD, 3>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 4: launch_o_t<HD, 4>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 5: launch_o_t<HD, 5>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 6: launch_o_t<HD, 6>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    case 7: launch_o_t<HD, 7>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
    default: launch_o_t<HD, 8>(otw, n_heads, qk, vt, wo, opart, scale_log2e, s); break;
  }
}

template <int HD, bool FRAG>
void launch_hd(int T, int n_heads, const half_t* qk, const half_t* vt, half_t* out, float scale_log2e,
               hipStream_t s) {
  switch (T / 64) {
    case 1: launch_t<HD, 1, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 2: launch_t<HD, 2, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 3: launch_t<HD, 3, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 4: launch_t<HD, 4, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 5: launch_t<HD, 5, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 6: launch_t<HD, 6, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    case 7: launch_t<HD, 7, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
    default: launch_t<HD, 8, FRAG>(n_heads, qk, vt, out, scale_log2e, s); break;
  }
}

}  // namespace

void launch_attention(const half_t* qk, const half_t* vt, half_t* out, int T, int n_heads, int head_dim, bool frag,
                      hipStream_t s) {
  CK_REQUIRE(qk && vt && out, "attention: null pointer");
  CK_REQUIRE(T > 0 && T % 64 == 0 && T <= ATT_TMAX, "attention: T must be a multiple of 64 and <= 512");
  CK_REQUIRE(head_dim == 64 || head_dim == 128, "attention: head_dim must be 64 or 128");
  CK_REQUIRE(n_heads > 0, "attention: n_heads must be positive");
  // the output leaves through raw buffer stores addressed by 32-bit offsets
  CK_REQUIRE(2L * T * n_heads * head_dim < (1L << 31), "attention: output must be under 2 GiB");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(qk) & 15) == 0 && (reinterpret_cast<uintptr_t>(vt) & 15) == 0 &&
                 (reinterpret_cast<uintptr_t>(out) & 7) == 0,
             "attention: qk and vt must be 16-byte and out 8-byte aligned");
  // scores go straight to the exp2 domain: s * (1/sqrt(hd)) * log2(e)
  const float scale_log2e = 1.4426950408889634f / sqrtf((float)head_dim);
  if (frag) {
    if (head_dim == 64) launch_hd<64, true>(T, n_heads, qk, vt, out, scale_log2e, s);
    else launch_hd<128, true>(T, n_heads, qk, vt, out, scale_log2e, s);
  } else {
    if (head_dim == 64) launch_hd<64, false>(T, n_heads, qk, vt, out, scale_log2e, s);
    else launch_hd<128, false>(T, n_heads, qk, vt, out, scale_log2e, s);
  }
  CK_LAUNCHED("attention");
}

int attention_oproj_tiles(int T, int n_heads, int head_dim) {
  if (T <= 0 || T % 64 != 0 || T > ATT_TMAX || (head_dim != 64 && head_dim != 128) || n_heads <= 0) return 0;
  const int tiles = n_heads * head_dim / 16, waves = att_waves(T / 64);
  if (tiles % waves != 0) return 0;
  const int otw = tiles / waves;
  return (otw == 1 || otw == 2 || otw == 4) ? otw : 0;
}

void launch_attention_oproj(const half_t* qk, const half_t* vt, const half_t* wo, float* opart, int T, int n_heads,
                            int head_dim, hipStream_t s) {
  CK_REQUIRE(qk && vt && wo && opart, "attention_oproj: null pointer");
  const int otw = attention_oproj_tiles(T, n_heads, head_dim);
  CK_REQUIRE(otw > 0,
             "attention_oproj: needs T a multiple of 64 up to 512, head_dim 64 or 128, and 1, 2 or 4 output "
             "tiles of 16 features per wave");
  CK_REQUIRE(4L * T * n_heads * head_dim < (1L << 31), "attention_oproj: partial plane too large");
  CK_REQUIRE(((reinterpret_cast<uintptr_t>(qk) | reinterpret_cast<uintptr_t>(vt) | reinterpret_cast<uintptr_t>(wo) |
               reinterpret_cast<uintptr_t>(opart)) & 15) == 0,
             "attention_oproj: operands must be 16-byte aligned");
  const float scale_log2e = 1.4426950408889634f / sqrtf((float)head_dim);
  if (head_dim == 64) launch_o_hd<64>(T, otw, n_heads, qk, vt, wo, opart, scale_log2e, s);
  else launch_o_hd<128>(T, otw, n_heads, qk, vt, wo, opart, scale_log2e, s);
  CK_LAUNCHED("attention_oproj");
}

}  // namespace ck
