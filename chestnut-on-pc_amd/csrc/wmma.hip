// Fragment-level known-answer kernels.
//
// wmma_rdna4: the reference's WMMA uop, ((16,16,16), half, 'AMD', 32)
// (run_pinned2.py:100-266), computed on gfx950.  The reference lowers it to
// FFMA chains or to four sm_75 mma.m16n8k8 ops through a shared-memory
// staging slice; here the 32 RDNA4 lanes' fragments are scattered into LDS
// matrices by the RDNA4 map and consumed by one v_mfma_f32_16x16x16_f16 of a
// 64-lane wave, with C as the MFMA accumulator input.
//   RDNA4 map (consumer_probe.py:14-19; run_pinned2.py:106-117):
//     element j of lane t holds k = j (+4 if t >= 16) for j < 4,
//                                  j + 4 (+4 if t >= 16) for j >= 4;
//     A[t%16][k], B[k][t%16]; D element e of lane t is D[(t/16)*8 + e][t%16].
//
// mfma_kat: one MFMA on plain row-major operands, written with the operand
// layout the GEMM and attention kernels assume, so a wrong layout shows up
// as a wrong product.
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

__device__ __forceinline__ int rdna4_k(int t, int j) {
  return j < 4 ? (t < 16 ? j : j + 4) : (t < 16 ? j + 4 : j + 8);
}

__global__ __launch_bounds__(64) void wmma_rdna4_kernel(const uint16_t* __restrict__ fa, const uint16_t* __restrict__ fb,
                                                        const float* __restrict__ fc, float* __restrict__ fd) {
  __shared__ uint16_t A[16][16], B[16][16];
  __shared__ float C[16][16], D[16][16];
  const int l = threadIdx.x;
  const long tile = blockIdx.x;
  fa += tile * 256; fb += tile * 256; fc += tile * 256; fd += tile * 256;
  if (l < 32) {
    for (int j = 0; j < 8; ++j) {
      const int k = rdna4_k(l, j);
      A[l % 16][k] = fa[l * 8 + j];
      B[k][l % 16] = fb[l * 8 + j];
      C[(l / 16) * 8 + j][l % 16] = fc[l * 8 + j];
    }
  }
  __syncthreads();
  // v_mfma_f32_16x16x16_f16: A row l%16, k = 4*(l/16)..+3; B column l%16, same k;
  // C/D element i of lane l is row 4*(l/16)+i, column l%16.
  half4_t a, b;
  float4_t c;
  for (int i = 0; i < 4; ++i) {
    a[i] = __builtin_bit_cast(half_t, A[l % 16][4 * (l / 16) + i]);
    b[i] = __builtin_bit_cast(half_t, B[4 * (l / 16) + i][l % 16]);
    c[i] = C[4 * (l / 16) + i][l % 16];
  }
  const float4_t d = __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  for (int i = 0; i < 4; ++i) D[4 * (l / 16) + i][l % 16] = d[i];
  __syncthreads();
  if (l < 32)
    for (int e = 0; e < 8; ++e) fd[l * 8 + e] = D[(l / 16) * 8 + e][l % 16];
}

__global__ __launch_bounds__(64) void mfma_kat_kernel(int variant, const uint16_t* __restrict__ A,
                                                      const uint16_t* __restrict__ B, float* __restrict__ D) {
  const int l = threadIdx.x;
  half8_t a, b;
  if (variant == 0) {   // 16x16x32: A [16][32], B [32][16]
    for (int j = 0; j < 8; ++j) {
      a[j] = __builtin_bit_cast(half_t, A[(l % 16) * 32 + 8 * (l / 16) + j]);
      b[j] = __builtin_bit_cast(half_t, B[(8 * (l / 16) + j) * 16 + l % 16]);
    }
    const float4_t acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, float4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    for (int i = 0; i < 4; ++i) D[(4 * (l / 16) + i) * 16 + l % 16] = acc[i];
  } else {              // 32x32x16: A [32][16], B [16][32]
    for (int j = 0; j < 8; ++j) {
      a[j] = __builtin_bit_cast(half_t, A[(l % 32) * 16 + 8 * (l / 32) + j]);
      b[j] = __builtin_bit_cast(half_t, B[(8 * (l / 32) + j) * 32 + l % 32]);
    }
    const float16_t acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, float16_t{}, 0, 0, 0);
    for (int e = 0; e < 16; ++e) D[(8 * (e / 4) + 4 * (l / 32) + e % 4) * 32 + l % 32] = acc[e];
  }
}

}  // namespace

void launch_wmma_rdna4(const uint16_t* fa, const uint16_t* fb, const float* fc, float* fd, int n_tiles,
                       hipStream_t s) {
  CK_REQUIRE(fa && fb && fc && fd && n_tiles > 0, "wmma_rdna4: bad arguments");
  CK_LAUNCH(wmma_rdna4_kernel, dim3(n_tiles), dim3(64), 0, s, fa, fb, fc, fd);
  CK_LAUNCHED("wmma_rdna4");
}

void launch_mfma_kat(int variant, const uint16_t* A, const uint16_t* B, float* D, hipStream_t s) {
  CK_REQUIRE(A && B && D, "mfma_kat: null pointer");
  CK_REQUIRE(variant == 0 || variant == 1, "mfma_kat: variant must be 0 (16x16x32) or 1 (32x32x16)");
  CK_LAUNCH(mfma_kat_kernel, dim3(1), dim3(64), 0, s, variant, A, B, D);
  CK_LAUNCHED("mfma_kat");
}

}  // namespace ck
