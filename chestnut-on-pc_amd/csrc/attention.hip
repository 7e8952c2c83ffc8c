// Non-causal multi-head attention for the token block of the driving model.
//
// The reference's attention lives in comma's pickle as WMMA GEMM kernels
// (NOTES.md:84-104); this is the gfx950 form of the same f16-input,
// f32-accumulate products with an f32 softmax between them.
//
// One workgroup = 32 queries of one head, 4 waves (T=512, 16 heads: 256
// workgroups, one per CU).  Every K and V element a workgroup needs is read
// by exactly one of its waves:
//   1. wave w computes S^T = K Q^T * scale for keys [w*T/4, (w+1)*T/4) and all
//      32 queries with v_mfma_f32_16x16x32_f16 (A = 16 keys x 32 head dims of
//      K, B = Q^T); the S^T tile stays in registers (T/8 floats per lane);
//   2. softmax per query: lane-local max / sum over its keys, xor-16/xor-32
//      lane exchanges, then the four waves' partials through a 1 KB LDS table
//      in fixed wave order (deterministic); P = e^(s-max) * (1/sum) rounded
//      to f16, with the hardware exp2 (v_exp_f32) and one reciprocal per
//      query: P is rounded to f16, far coarser than either approximation, and
//      the exact exp and a division per element cost 2.4 us of a 10.6 us launch
//      into LDS as P[query][key] (the D layout gives each lane four
//      consecutive keys of one query: one 8-byte LDS write);
//   3. wave w computes O[:, w*hd/4 .. +hd/4) = P V over all T keys: A = P from
//      LDS (rows padded to T+8 halves: the 16 rows a 16-lane group reads fall
//      in distinct banks), B = V^T [d][T] (written transposed by the QKV GEMM
//      epilogue) so a lane's 8 consecutive keys are one 16-byte load.
// Workgroups are regrouped by XCD (consecutive ids land on different XCDs):
// each XCD's L2 then serves the K/V of T*hd*2*2 bytes for 2 heads.
// MFMA 16x16x32 layout (lane l): A row l%16, k = 8*(l/16)..+7; B column
// l%16, same k; D element i of lane l is row 4*(l/16)+i, column l%16.
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

// NKT = T / 64; WAVES = 8 (hd 128, T % 128 == 0) or 4.  Every load a wave
// makes (its Q fragments, its T/WAVES keys, its hd/WAVES columns of V^T) is
// issued at entry, before any MFMA: the K/V working set of a workgroup
// (T*hd*2*2 bytes) is then in flight at once instead of a few loads per
// wave, which is what bounds a one-workgroup-per-CU kernel on data that
// comes from the Infinity Cache.
// FRAG: qk / vt hold the operands in MFMA fragment order (written by the
// QKV GEMM's fragment epilogue): every fragment load of a wave is one
// contiguous KB.  Otherwise the row layouts: qk [T][2d], vt [d][T].
template <int HD, int NKT, int WAVES, bool FRAG>
__global__ __launch_bounds__(64 * WAVES) void attention_kernel(const half_t* __restrict__ qk,
                                                               const half_t* __restrict__ vt,
                                                               half_t* __restrict__ out, int n_heads, float scale) {
  constexpr int T = 64 * NKT;
  constexpr int KS = HD / 32;        // k-steps of the q.k products
  constexpr int KPW = T / WAVES;     // keys per wave in phase 1
  constexpr int KT = KPW / 16;       // 16-key tiles per wave
  constexpr int CW = HD / WAVES;     // output columns per wave in phase 3
  constexpr int CT = CW / 16;        // 16-wide output tiles per wave
  constexpr int NT = T / 32;         // 32-key steps of phase 3
  constexpr int LP = T + 8;          // P row pitch (halves)
  static_assert(KPW % 16 == 0 && CW % 16 == 0, "wave split must keep whole MFMA tiles");
  __shared__ __attribute__((aligned(16))) half_t P[ATT_QB][LP];
  __shared__ float red[2][WAVES][ATT_QB];

  const int d = n_heads * HD;
  const int nqb = T / ATT_QB;
  const int total = nqb * n_heads;
  int L = blockIdx.x;
  if ((total & 7) == 0) L = (L & 7) * (total >> 3) + (L >> 3);
  const int h = L / nqb, q0 = (L % nqb) * ATT_QB;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const long ldq = 2L * d;
  const int kw0 = wave * KPW;

  // ---- all loads up front ----
  half8_t qf[2][KS], kf[KT][KS], vb[NT][CT];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[kt][ks] = *reinterpret_cast<const half8_t*>(
          FRAG ? qk + ((((long)(n_heads + h) * (T / 16) + kw0 / 16 + kt) * KS + ks) * 64 + lane) * 8
               : qk + (long)(kw0 + kt * 16 + r16) * ldq + d + h * HD + ks * 32 + g * 8);
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[qt][ks] = *reinterpret_cast<const half8_t*>(
          FRAG ? qk + ((((long)h * (T / 16) + q0 / 16 + qt) * KS + ks) * 64 + lane) * 8
               : qk + (long)(q0 + qt * 16 + r16) * ldq + h * HD + ks * 32 + g * 8);
  const half_t* vrow = vt + (long)(h * HD + wave * CW + r16) * T + g * 8;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
      vb[t][ct] = *reinterpret_cast<const half8_t*>(
          FRAG ? vt + ((((long)h * (HD / 16) + wave * CT + ct) * NT + t) * 64 + lane) * 8
               : vrow + (long)ct * 16 * T + t * 32);

  // ---- phase 1: S^T = K Q^T for this wave's keys ----
  float4_t s[KT][2];
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
      float4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf[kt][ks], qf[qt][ks], a, 0, 0, 0);
      s[kt][qt] = a * scale;
    }

  // ---- phase 2: softmax per query (column r16 of q-tile qt) ----
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    float m = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) m = fmaxf(m, s[kt][qt][i]);
    m = xor_max(m);
    if (g == 0) red[0][wave][qt * 16 + r16] = m;
  }
  __syncthreads();
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = qt * 16 + r16;
    float mx = red[0][0][q];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) mx = fmaxf(mx, red[0][w][q]);
    float acc = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = __expf(s[kt][qt][i] - mx);   // v_exp_f32 on (s - max) * log2(e)
        s[kt][qt][i] = e;
        acc += e;
      }
    acc = xor_sum(acc);
    if (g == 0) red[1][wave][q] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int q = qt * 16 + r16;
    float sum = red[1][0][q];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) sum += red[1][w][q];
    const float rs = 1.0f / sum;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      half4_t pv;
#pragma unroll
      for (int i = 0; i < 4; ++i) pv[i] = (half_t)(s[kt][qt][i] * rs);
      *reinterpret_cast<half4_t*>(&P[q][kw0 + kt * 16 + 4 * g]) = pv;
    }
  }
  __syncthreads();

  // ---- phase 3: O[:, wave's columns] = P V ----
  float4_t o[2][CT];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) o[qt][ct] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    half8_t pa[2];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) pa[qt] = *reinterpret_cast<const half8_t*>(&P[qt * 16 + r16][t * 32 + g * 8]);
#pragma unroll
    for (int qt = 0; qt < 2; ++qt)
#pragma unroll
      for (int ct = 0; ct < CT; ++ct)
        o[qt][ct] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa[qt], vb[t][ct], o[qt][ct], 0, 0, 0);
  }
#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        out[(long)(q0 + qt * 16 + 4 * g + i) * d + h * HD + wave * CW + ct * 16 + r16] = (half_t)o[qt][ct][i];
}

template <int HD, int NKT, bool FRAG>
void launch_t(int n_heads, const half_t* qk, const half_t* vt, half_t* out, float scale, hipStream_t s) {
  const dim3 grid((64 * NKT / ATT_QB) * n_heads);
  if constexpr (HD == 128 && NKT % 2 == 0)
    hipLaunchKernelGGL((attention_kernel<HD, NKT, 8, FRAG>), grid, dim3(512), 0, s, qk, vt, out, n_heads, scale);
  else
    hipLaunchKernelGGL((attention_kernel<HD, NKT, 4, FRAG>), grid, dim3(256), 0, s, qk, vt, out, n_heads, scale);
}

template <int HD, bool FRAG>
void launch_hd(int T, int n_heads, const half_t* qk, const half_t* vt, half_t* out, float scale, hipStream_t s) {
  switch (T / 64) {
    case 1: launch_t<HD, 1, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 2: launch_t<HD, 2, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 3: launch_t<HD, 3, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 4: launch_t<HD, 4, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 5: launch_t<HD, 5, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 6: launch_t<HD, 6, FRAG>(n_heads, qk, vt, out, scale, s); break;
    case 7: launch_t<HD, 7, FRAG>(n_heads, qk, vt, out, scale, s); break;
    default: launch_t<HD, 8, FRAG>(n_heads, qk, vt, out, scale, s); break;
  }
}

}  // namespace

void launch_attention(const half_t* qk, const half_t* vt, half_t* out, int T, int n_heads, int head_dim, bool frag,
                      hipStream_t s) {
  CK_REQUIRE(qk && vt && out, "attention: null pointer");
  CK_REQUIRE(T > 0 && T % 64 == 0 && T <= ATT_TMAX, "attention: T must be a multiple of 64 and <= 512");
  CK_REQUIRE(head_dim == 64 || head_dim == 128, "attention: head_dim must be 64 or 128");
  CK_REQUIRE(n_heads > 0, "attention: n_heads must be positive");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(qk) & 15) == 0 && (reinterpret_cast<uintptr_t>(vt) & 15) == 0,
             "attention: qk and vt must be 16-byte aligned");
  const float scale = 1.0f / sqrtf((float)head_dim);
  if (frag) {
    if (head_dim == 64) launch_hd<64, true>(T, n_heads, qk, vt, out, scale, s);
    else launch_hd<128, true>(T, n_heads, qk, vt, out, scale, s);
  } else {
    if (head_dim == 64) launch_hd<64, false>(T, n_heads, qk, vt, out, scale, s);
    else launch_hd<128, false>(T, n_heads, qk, vt, out, scale, s);
  }
  CK_LAUNCHED("attention");
}

}  // namespace ck
