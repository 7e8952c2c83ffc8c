// Row LayerNorm, token mean-pool, GRU gate, token-embedding init and the
// end-of-frame tick.  All HBM-bound elementwise / row kernels; one wave per
// row where a reduction is needed (DPP wave reductions, no LDS).
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

// One wave per row; EPL = d / 64 elements per lane, read lane-strided so
// every load instruction of the wave covers 256 contiguous bytes.
template <int EPL, bool OUT_F16>
__global__ __launch_bounds__(256) void layernorm_kernel(const float* __restrict__ x, const float* __restrict__ g,
                                                        const float* __restrict__ b, void* __restrict__ out, int rows,
                                                        float eps) {
  constexpr int D = EPL * 64;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;   // whole wave leaves together; no barriers below
  const float* xr = x + (long)row * D;
  float v[EPL];
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < EPL; ++i) {
    v[i] = xr[lane + 64 * i];
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

template <int EPL>
void ln_launch(const float* x, const float* g, const float* b, void* out, bool f16, int rows, float eps,
               hipStream_t s) {
  dim3 grid((rows + 3) / 4);
  if (f16) hipLaunchKernelGGL((layernorm_kernel<EPL, true>), grid, dim3(256), 0, s, x, g, b, out, rows, eps);
  else hipLaunchKernelGGL((layernorm_kernel<EPL, false>), grid, dim3(256), 0, s, x, g, b, out, rows, eps);
  CK_LAUNCHED("layernorm");
}

// out[n] = (1/rows) * sum_t x[t][n], summed in row order (deterministic).
__global__ __launch_bounds__(256) void colmean_kernel(const float* __restrict__ x, float* __restrict__ out, int rows,
                                                      int d) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= d) return;
  float s = 0.f;
  for (int t = 0; t < rows; ++t) s += x[(long)t * d + n];
  out[n] = s / (float)rows;
}

// GRU update (gate order r, z, n as rows [0,H), [H,2H), [2H,3H)):
// r = sig(gi_r + gh_r), z = sig(gi_z + gh_z), n = tanh(gi_n + r * gh_n),
// h = (1 - z) * n + z * h_prev.  gi, gh already include their biases.
__global__ __launch_bounds__(256) void gru_gate_kernel(const float* __restrict__ gi, const float* __restrict__ gh,
                                                       const float* __restrict__ hp, float* __restrict__ h1,
                                                       float* __restrict__ h2, int H) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= H) return;
  const float r = sigmoidf_(gi[j] + gh[j]);
  const float z = sigmoidf_(gi[H + j] + gh[H + j]);
  const float n = tanhf(gi[2 * H + j] + r * gh[2 * H + j]);
  const float h = (1.0f - z) * n + z * hp[j];
  h1[j] = h;
  if (h2) h2[j] = h;
}

// X[t][n] = pos[t][n] + ctx[n] + bias[n] (the embedding GEMM then adds F W^T).
__global__ __launch_bounds__(256) void embed_init_kernel(const half_t* __restrict__ pos, const float* __restrict__ ctx,
                                                         const float* __restrict__ bias, float* __restrict__ X, int T,
                                                         int d) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)T * d) return;
  const int n = (int)(i % d);
  X[i] = ((float)pos[i] + ctx[n]) + bias[n];
}

// End of frame: advance the queue frame counter and feed the new hidden
// state back into the packed input's prev_feat slot (the host recurrence of
// run_pinned2.py:1580, done on device so back-to-back frames need no host).
__global__ __launch_bounds__(256) void frame_tick_kernel(unsigned* counter, const float* __restrict__ h,
                                                         float* __restrict__ feat, int H) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j == 0) counter[0] = counter[0] + 1u;
  if (j < H) feat[j] = h[j];
}

__global__ __launch_bounds__(256) void fill_u32_kernel(unsigned* p, unsigned v, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

void launch_layernorm(const float* x, const float* g, const float* b, void* out, bool out_f16, int rows, int d,
                      float eps, hipStream_t s) {
  CK_REQUIRE(x && g && b && out && rows > 0, "layernorm: bad arguments");
  switch (d) {
    case 128: ln_launch<2>(x, g, b, out, out_f16, rows, eps, s); break;
    case 256: ln_launch<4>(x, g, b, out, out_f16, rows, eps, s); break;
    case 512: ln_launch<8>(x, g, b, out, out_f16, rows, eps, s); break;
    case 1024: ln_launch<16>(x, g, b, out, out_f16, rows, eps, s); break;
    case 2048: ln_launch<32>(x, g, b, out, out_f16, rows, eps, s); break;
    default: throw Error("layernorm: d must be one of 128, 256, 512, 1024, 2048");
  }
}

void launch_colmean(const float* x, float* out, int rows, int d, hipStream_t s) {
  CK_REQUIRE(x && out && rows > 0 && d > 0, "colmean: bad arguments");
  hipLaunchKernelGGL(colmean_kernel, dim3(ceil_div(d, 256)), dim3(256), 0, s, x, out, rows, d);
  CK_LAUNCHED("colmean");
}

void launch_gru_gate(const float* gi, const float* gh, const float* h_prev, float* h_out, float* h_out2, int H,
                     hipStream_t s) {
  CK_REQUIRE(gi && gh && h_prev && h_out && H > 0, "gru_gate: bad arguments");
  hipLaunchKernelGGL(gru_gate_kernel, dim3(ceil_div(H, 256)), dim3(256), 0, s, gi, gh, h_prev, h_out, h_out2, H);
  CK_LAUNCHED("gru_gate");
}

void launch_embed_init(const half_t* pos, const float* ctx, const float* bias, float* X, int T, int d,
                       hipStream_t s) {
  CK_REQUIRE(pos && ctx && bias && X, "embed_init: null pointer");
  hipLaunchKernelGGL(embed_init_kernel, dim3(ceil_div((long)T * d, 256)), dim3(256), 0, s, pos, ctx, bias, X, T, d);
  CK_LAUNCHED("embed_init");
}

void launch_frame_tick(unsigned* counter, const float* h, float* packed_feat, int H, hipStream_t s) {
  hipLaunchKernelGGL(frame_tick_kernel, dim3(ceil_div(H, 256)), dim3(256), 0, s, counter, h, packed_feat, H);
  CK_LAUNCHED("frame_tick");
}

void launch_fill_u32(void* p, unsigned v, size_t n_words, hipStream_t s) {
  if (n_words == 0) return;
  hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)((n_words + 255) / 256)), dim3(256), 0, s,
                     static_cast<unsigned*>(p), v, n_words);
  CK_LAUNCHED("fill_u32");
}

}  // namespace ck
