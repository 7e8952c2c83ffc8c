// Row LayerNorm (with the residual update of a split-K GEMM folded in), the
// token mean-pool and a fill kernel.  HBM-bound row kernels: DPP wave
// reductions, and for wide rows the four wave sums through LDS.
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

// One wave per row; EPL = d / 64 elements per lane, read lane-strided so
// every load instruction of the wave covers 256 contiguous bytes.
// ADD: the row first takes the residual update of the preceding split-K
// GEMM, x += ((ws[0] + ws[1]) + ... + ws[S-1]) + bias, written back to x.
template <int EPL, bool OUT_F16, bool ADD>
__global__ __launch_bounds__(256) void layernorm_kernel(float* __restrict__ x, const float* __restrict__ ws, int nsplit,
                                                        long split_stride, const float* __restrict__ rbias,
                                                        const float* __restrict__ g, const float* __restrict__ b,
                                                        void* __restrict__ out, int rows, float eps) {
  constexpr int D = EPL * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;   // whole wave leaves together; no barriers below
  float* xr = x + (long)row * D;
  float v[EPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int c = lane + 64 * i;
    v[i] = xr[c];
    if (ADD) {
      const float* w = ws + (long)row * D + c;
      float a = w[0];
      for (int k = 1; k < nsplit; ++k) a += w[k * split_stride];
      if (rbias) a += rbias[c];
      v[i] = v[i] + a;
      xr[c] = v[i];
    }
    s += v[i];
  }
  const float mean = wave_sum(s) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const float c = v[i] - mean;
    q = fmaf(c, c, q);
  }
  const float var = wave_sum(q) / (float)D;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    const int c = lane + 64 * i;
    const float y = (v[i] - mean) * rstd * g[c] + b[c];
    if (OUT_F16) static_cast<half_t*>(out)[(long)row * D + c] = (half_t)y;
    else static_cast<float*>(out)[(long)row * D + c] = y;
  }
}

// Wide rows (d >= 1024; d = 512 has the wave form below): one 256-thread
// workgroup per row.  Thread t owns the VW-wide chunks t, t+256, ... (VW = 4,
// or 2 for d = 512), so every access is a coalesced 8/16-byte vector.  All loads -- x, every split-K partial (up to
// LN_MAXS), the bias, gamma and beta -- are issued before any arithmetic: one
// memory round trip per row instead of one per partial.  Per element the
// residual update is x + ((((ws0 + ws1) + ws2) + ...) + bias), in split
// order.  Row sums: DPP wave sums, then the 4 wave sums through LDS in order.
// With 16-byte chunks (d >= 1024) the updated x and the f16 output, both read
// by the next kernel, leave with the device-scope cache policy (store_sc1;
// -1.1% of the 1B frame against default stores).
constexpr int LN_MAXS = 8;

// NS: 0 no residual update; > 0 exactly NS partials (loads unconditional);
// -1 up to LN_MAXS partials, count at run time.
template <int EPT, bool OUT_F16, int NS>
__global__ __launch_bounds__(256) void layernorm_row_kernel(float* __restrict__ x, const float* __restrict__ ws,
                                                            int nsplit, long split_stride,
                                                            const float* __restrict__ rbias,
                                                            const float* __restrict__ g, const float* __restrict__ b,
                                                            void* __restrict__ out, float eps) {
  constexpr int D = EPT * 256;
  constexpr int VW = EPT >= 4 ? 4 : EPT;
  constexpr int NV = EPT / VW;
  typedef float vec_t __attribute__((ext_vector_type(VW)));
  typedef _Float16 hvec_t __attribute__((ext_vector_type(VW)));
  __shared__ float red[2][4];
  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  float* xr = x + (long)row * D;
  vec_t v[NV], gv[NV], bv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 256 + tid) * VW;
    v[j] = *reinterpret_cast<const vec_t*>(xr + c);
    gv[j] = *reinterpret_cast<const vec_t*>(g + c);
    bv[j] = *reinterpret_cast<const vec_t*>(b + c);
  }
  if (NS != 0) {
    constexpr int KN = NS > 0 ? NS : LN_MAXS;
    vec_t p[KN][NV], rb[NV];
    const float* w = ws + (long)row * D;
#pragma unroll
    for (int k = 0; k < KN; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j)
        p[k][j] = (NS > 0 || k < nsplit) ? *reinterpret_cast<const vec_t*>(w + k * split_stride + (j * 256 + tid) * VW)
                                         : vec_t{};
#pragma unroll
    for (int j = 0; j < NV; ++j)
      rb[j] = rbias ? *reinterpret_cast<const vec_t*>(rbias + (j * 256 + tid) * VW) : vec_t{};
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      vec_t a = p[0][j];
#pragma unroll
      for (int k = 1; k < KN; ++k)
        if (NS > 0 || k < nsplit) a += p[k][j];
      if (rbias) a += rb[j];
      v[j] = v[j] + a;
      if constexpr (VW == 4) store_sc1(sc1_rsrc(xr, 4L * D), 4L * (j * 256 + tid) * VW, v[j]);
      else *reinterpret_cast<vec_t*>(xr + (j * 256 + tid) * VW) = v[j];
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VW; ++e) s += v[j][e];
  s = wave_sum(s);
  if (lane == 0) red[0][wave] = s;
  __syncthreads();
  const float mean = (((red[0][0] + red[0][1]) + red[0][2]) + red[0][3]) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      const float c = v[j][e] - mean;
      q = fmaf(c, c, q);
    }
  q = wave_sum(q);
  if (lane == 0) red[1][wave] = q;
  __syncthreads();
  const float var = (((red[1][0] + red[1][1]) + red[1][2]) + red[1][3]) / (float)D;
  const float rstd = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const long c = (long)row * D + (j * 256 + tid) * VW;
    vec_t y;
#pragma unroll
    for (int e = 0; e < VW; ++e) y[e] = (v[j][e] - mean) * rstd * gv[j][e] + bv[j][e];
    if (OUT_F16) {
      hvec_t h;
#pragma unroll
      for (int e = 0; e < VW; ++e) h[e] = (half_t)y[e];
      if constexpr (VW == 4) store_sc1(sc1_rsrc(static_cast<half_t*>(out) + (long)row * D, 2L * D), 2L * (c - (long)row * D), h);
      else *reinterpret_cast<hvec_t*>(static_cast<half_t*>(out) + c) = h;
    } else {
      if constexpr (VW == 4) store_sc1(sc1_rsrc(static_cast<float*>(out) + (long)row * D, 4L * D), 4L * (c - (long)row * D), y);
      else *reinterpret_cast<vec_t*>(static_cast<float*>(out) + c) = y;
    }
  }
}

// d = 512 (the 39M model): one 64-lane wave per row, a workgroup each.
// Lane l owns the 16-byte chunks l and l + 64, loaded with every partial,
// the bias, gamma and beta before any arithmetic; the same per-element
// residual order as the row kernel; row sums by DPP wave sums alone (no LDS,
// no barrier).
template <bool OUT_F16, int NS>
__global__ __launch_bounds__(64) void layernorm_wave_kernel(float* __restrict__ x, const float* __restrict__ ws,
                                                            int nsplit, long split_stride,
                                                            const float* __restrict__ rbias,
                                                            const float* __restrict__ g, const float* __restrict__ b,
                                                            void* __restrict__ out, float eps) {
  constexpr int NV = 2, D = NV * 256;
  const int row = blockIdx.x, lane = threadIdx.x;
  float* xr = x + (long)row * D;
  float4_t v[NV], gv[NV], bv[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    v[j] = *reinterpret_cast<const float4_t*>(xr + c);
    gv[j] = *reinterpret_cast<const float4_t*>(g + c);
    bv[j] = *reinterpret_cast<const float4_t*>(b + c);
  }
  if (NS != 0) {
    constexpr int KN = NS > 0 ? NS : LN_MAXS;
    float4_t p[KN][NV], rb[NV];
    const float* w = ws + (long)row * D;
#pragma unroll
    for (int k = 0; k < KN; ++k)
#pragma unroll
      for (int j = 0; j < NV; ++j)
        p[k][j] = (NS > 0 || k < nsplit) ? *reinterpret_cast<const float4_t*>(w + k * split_stride + (j * 64 + lane) * 4)
                                         : float4_t{};
#pragma unroll
    for (int j = 0; j < NV; ++j) rb[j] = rbias ? *reinterpret_cast<const float4_t*>(rbias + (j * 64 + lane) * 4) : float4_t{};
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      float4_t a = p[0][j];
#pragma unroll
      for (int k = 1; k < KN; ++k)
        if (NS > 0 || k < nsplit) a += p[k][j];
      if (rbias) a += rb[j];
      v[j] = v[j] + a;
      store_sc1(sc1_rsrc(xr, 4L * D), 4L * (j * 64 + lane) * 4, v[j]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) s += (v[j][0] + v[j][1]) + (v[j][2] + v[j][3]);
  const float mean = wave_sum(s) / (float)D;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float c = v[j][e] - mean;
      q = fmaf(c, c, q);
    }
  const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)D + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * 64 + lane) * 4;
    float4_t y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = (v[j][e] - mean) * rstd * gv[j][e] + bv[j][e];
    if (OUT_F16)
      store_sc1(sc1_rsrc(static_cast<half_t*>(out) + (long)row * D, 2L * D), 2L * c,
                half4_t{(half_t)y[0], (half_t)y[1], (half_t)y[2], (half_t)y[3]});
    else
      store_sc1(sc1_rsrc(static_cast<float*>(out) + (long)row * D, 4L * D), 4L * c, y);
  }
}

void ln_wave_launch(float* x, const float* ws, int nsplit, long sstride, const float* rbias, const float* g,
                    const float* b, void* out, bool f16, int rows, float eps, hipStream_t s) {
  auto go = [&](auto ns) {
    constexpr int NS = decltype(ns)::value;
    if (f16) CK_LAUNCH((layernorm_wave_kernel<true, NS>), dim3(rows), dim3(64), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, eps);
    else CK_LAUNCH((layernorm_wave_kernel<false, NS>), dim3(rows), dim3(64), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, eps);
  };
  if (!ws) go(std::integral_constant<int, 0>{});
  else if (nsplit == 1) go(std::integral_constant<int, 1>{});
  else if (nsplit == 2) go(std::integral_constant<int, 2>{});
  else if (nsplit == 4) go(std::integral_constant<int, 4>{});
  else if (nsplit == 8) go(std::integral_constant<int, 8>{});
  else go(std::integral_constant<int, -1>{});
  CK_LAUNCHED("layernorm_wave");
}

template <int EPT>
void ln_row_launch(float* x, const float* ws, int nsplit, long sstride, const float* rbias, const float* g,
                   const float* b, void* out, bool f16, int rows, float eps, hipStream_t s) {
  dim3 grid(rows);
  auto go = [&](auto ns) {
    constexpr int NS = decltype(ns)::value;
    if (f16) CK_LAUNCH((layernorm_row_kernel<EPT, true, NS>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, eps);
    else CK_LAUNCH((layernorm_row_kernel<EPT, false, NS>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, eps);
  };
  if (!ws) go(std::integral_constant<int, 0>{});
  else if (nsplit == 1) go(std::integral_constant<int, 1>{});
  else if (nsplit == 2) go(std::integral_constant<int, 2>{});
  else if (nsplit == 4) go(std::integral_constant<int, 4>{});
  else go(std::integral_constant<int, -1>{});
  CK_LAUNCHED("layernorm_row");
}

template <int EPL>
void ln_launch(float* x, const float* ws, int nsplit, long sstride, const float* rbias, const float* g, const float* b,
               void* out, bool f16, int rows, float eps, hipStream_t s) {
  dim3 grid((rows + 3) / 4);
  if (ws) {
    if (f16) CK_LAUNCH((layernorm_kernel<EPL, true, true>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, rows, eps);
    else CK_LAUNCH((layernorm_kernel<EPL, false, true>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, rows, eps);
  } else {
    if (f16) CK_LAUNCH((layernorm_kernel<EPL, true, false>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, rows, eps);
    else CK_LAUNCH((layernorm_kernel<EPL, false, false>), grid, dim3(256), 0, s, x, ws, nsplit, sstride, rbias, g, b, out, rows, eps);
  }
  CK_LAUNCHED("layernorm");
}

// Column mean (mean-pool over tokens) in one deterministic pass.  A block of
// 256 threads owns 32 columns: thread t sums rows t/8, t/8 + 32, ... of the
// 4 columns 4*(t%8) .. +3 (all of its float4 loads issued before the adds,
// 16 in flight at 512 rows), then the 32 row-slice sums of each column are
// added through LDS in slice order and divided by the row count.  d = 2048
// gives 64 blocks.
constexpr int COLMEAN_COLS = 32;
constexpr int COLMEAN_BATCH = 16;   // loads in flight per thread

__global__ __launch_bounds__(256) void colmean_kernel(const float* __restrict__ x, float* __restrict__ out, int rows,
                                                      int d) {
  __shared__ float red[32][COLMEAN_COLS + 1];
  const int t = threadIdx.x, cg = t & 7, rs = t >> 3;
  const int c = blockIdx.x * COLMEAN_COLS + cg * 4;
  float4_t s = {0.f, 0.f, 0.f, 0.f};
  for (int r0 = rs; r0 < rows; r0 += 32 * COLMEAN_BATCH) {
    float4_t v[COLMEAN_BATCH];
#pragma unroll
    for (int k = 0; k < COLMEAN_BATCH; ++k) {
      const int r = r0 + 32 * k;
      v[k] = r < rows ? *reinterpret_cast<const float4_t*>(x + (long)r * d + c) : float4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < COLMEAN_BATCH; ++k) s += v[k];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) red[rs][cg * 4 + e] = s[e];
  __syncthreads();
  if (t < COLMEAN_COLS) {
    float a = 0.f;
#pragma unroll 8
    for (int i = 0; i < 32; ++i) a += red[i][t];
    out[blockIdx.x * COLMEAN_COLS + t] = a / (float)rows;
  }
}

__global__ __launch_bounds__(256) void fill_u32_kernel(unsigned* p, unsigned v, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

void launch_layernorm(const float* x, const float* g, const float* b, void* out, bool out_f16, int rows, int d,
                      float eps, hipStream_t s) {
  launch_add_layernorm(const_cast<float*>(x), nullptr, 0, 0, nullptr, g, b, out, out_f16, rows, d, eps, s);
}

void launch_add_layernorm(float* x, const float* ws, int nsplit, long split_stride, const float* rbias, const float* g,
                          const float* b, void* out, bool out_f16, int rows, int d, float eps, hipStream_t s) {
  CK_REQUIRE(x && g && b && out && rows > 0, "layernorm: bad arguments");
  CK_REQUIRE(!ws || (nsplit >= 1 && nsplit <= LN_MAXS), "layernorm: residual partials need 1 <= nsplit <= 8");
  if (d >= 512)
    CK_REQUIRE(((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(ws) | reinterpret_cast<uintptr_t>(rbias) |
                 reinterpret_cast<uintptr_t>(g) | reinterpret_cast<uintptr_t>(b) | reinterpret_cast<uintptr_t>(out)) &
                15) == 0 && split_stride % 4 == 0,
               "layernorm: wide rows need 16-byte aligned operands and a partial stride of whole vectors");
  switch (d) {
    case 128: ln_launch<2>(x, ws, nsplit, split_stride, rbias, g, b, out, out_f16, rows, eps, s); break;
    case 256: ln_launch<4>(x, ws, nsplit, split_stride, rbias, g, b, out, out_f16, rows, eps, s); break;
    case 512: ln_wave_launch(x, ws, nsplit, split_stride, rbias, g, b, out, out_f16, rows, eps, s); break;
    case 1024: ln_row_launch<4>(x, ws, nsplit, split_stride, rbias, g, b, out, out_f16, rows, eps, s); break;
    case 2048: ln_row_launch<8>(x, ws, nsplit, split_stride, rbias, g, b, out, out_f16, rows, eps, s); break;
    default: throw Error("layernorm: d must be one of 128, 256, 512, 1024, 2048");
  }
}

void launch_colmean(const float* x, float* out, int rows, int d, hipStream_t s) {
  CK_REQUIRE(x && out && rows > 0 && d > 0, "colmean: bad arguments");
  CK_REQUIRE(d % COLMEAN_COLS == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0,
             "colmean: d must be a multiple of 32 and x 16-byte aligned");
  CK_LAUNCH(colmean_kernel, dim3(d / COLMEAN_COLS), dim3(256), 0, s, x, out, rows, d);
  CK_LAUNCHED("colmean");
}

void launch_fill_u32(void* p, unsigned v, size_t n_words, hipStream_t s) {
  if (n_words == 0) return;
  CK_LAUNCH(fill_u32_kernel, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0, s,
                     static_cast<unsigned*>(p), v, n_words);
  CK_LAUNCHED("fill_u32");
}

}  // namespace ck
