// Non-causal multi-head attention for the token block of the driving model.
//
// The reference's attention lives in comma's pickle as WMMA GEMM kernels
// (NOTES.md:84-104); this is the gfx950 form of the same f16-input,
// f32-accumulate products with an f32 softmax between them.
//
// One workgroup = 16 query rows of one head, 4 waves:
//   1. S = q k^T * scale: each wave takes T/4 keys in 16-key blocks,
//      v_mfma_f32_16x16x32_f16 with q fragments held in registers and k read
//      straight from the packed QK tensor (16 bytes per lane); S -> LDS (f32).
//   2. softmax per row in f32 (max, exp, sum via DPP wave reductions), the
//      normalised probabilities rounded to f16 into LDS.
//   3. O = P v: v arrives transposed (V^T [d][T], written by the QKV GEMM
//      epilogue) so each lane's 8 consecutive keys are one 16-byte load.
// MFMA 16x16x32 layout (lane l): A row l%16, k = 8*(l/16)..+7; B column
// l%16, same k; D element i of lane l is row 4*(l/16)+i, column l%16.
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

constexpr int ATT_TMAX = 512;
constexpr int ATT_LS = ATT_TMAX + 4;
constexpr int ATT_LP = ATT_TMAX + 8;

template <int HD>
__global__ __launch_bounds__(256) void attention_kernel(const half_t* __restrict__ qk, const half_t* __restrict__ vt,
                                                        half_t* __restrict__ out, int T, int d, float scale) {
  __shared__ float S[16][ATT_LS];
  __shared__ __attribute__((aligned(16))) half_t P[16][ATT_LP];
  const int h = blockIdx.y, q0 = blockIdx.x * 16;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g = lane >> 4;
  const long ldq = 2L * d;

  constexpr int KS = HD / 32;
  half8_t qf[KS];
  const half_t* qrow = qk + (long)(q0 + r16) * ldq + h * HD + g * 8;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const half8_t*>(qrow + ks * 32);

  const int kpw = T / 4;
  for (int kb = wave * kpw; kb < (wave + 1) * kpw; kb += 16) {
    const half_t* krow = qk + (long)(kb + r16) * ldq + d + h * HD + g * 8;
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(qf[ks], *reinterpret_cast<const half8_t*>(krow + ks * 32), acc, 0,
                                                  0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) S[4 * g + i][kb + r16] = acc[i] * scale;
  }
  __syncthreads();

  constexpr int NPL = ATT_TMAX / 64;
  for (int rr = 0; rr < 4; ++rr) {
    const int r = wave * 4 + rr;
    float v[NPL];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = lane + 64 * i;
      v[i] = c < T ? S[r][c] : -INFINITY;
      mx = fmaxf(mx, v[i]);
    }
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = lane + 64 * i;
      v[i] = c < T ? expf(v[i] - mx) : 0.f;
      sum += v[i];
    }
    sum = wave_sum(sum);
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
      const int c = lane + 64 * i;
      if (c < T) P[r][c] = (half_t)(v[i] / sum);
    }
  }
  __syncthreads();

  for (int cb = wave; cb < HD / 16; cb += 4) {
    float4_t acc = {0.f, 0.f, 0.f, 0.f};
    const half_t* vrow = vt + (long)(h * HD + cb * 16 + r16) * T + g * 8;
    for (int k = 0; k < T; k += 32) {
      const half8_t pa = *reinterpret_cast<const half8_t*>(&P[r16][k + g * 8]);
      const half8_t vb = *reinterpret_cast<const half8_t*>(vrow + k);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) out[(long)(q0 + 4 * g + i) * d + h * HD + cb * 16 + r16] = (half_t)acc[i];
  }
}

}  // namespace

void launch_attention(const half_t* qk, const half_t* vt, half_t* out, int T, int n_heads, int head_dim,
                      hipStream_t s) {
  CK_REQUIRE(qk && vt && out, "attention: null pointer");
  CK_REQUIRE(T > 0 && T % 64 == 0 && T <= ATT_TMAX, "attention: T must be a multiple of 64 and <= 512");
  CK_REQUIRE(head_dim == 64 || head_dim == 128, "attention: head_dim must be 64 or 128");
  CK_REQUIRE(n_heads > 0, "attention: n_heads must be positive");
  const int d = n_heads * head_dim;
  const float scale = 1.0f / sqrtf((float)head_dim);
  dim3 grid(T / 16, n_heads);
  if (head_dim == 64)
    hipLaunchKernelGGL(attention_kernel<64>, grid, dim3(256), 0, s, qk, vt, out, T, d, scale);
  else
    hipLaunchKernelGGL(attention_kernel<128>, grid, dim3(256), 0, s, qk, vt, out, T, d, scale);
  CK_LAUNCHED("attention");
}

}  // namespace ck
