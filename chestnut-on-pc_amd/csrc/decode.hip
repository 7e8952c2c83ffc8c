// Output decode of the frame: the device form of the reference's host-side
// Parser (parse_model_outputs.py:4-120), run as the last entries of the
// frame plan so the parsed heads are ready with the raw output vector.
//
// One workgroup per output head; the head's kind comes from the Parser's
// name table (the engine resolves it, see engine.cpp build_decode):
//   RAW      copy (heads the Parser does not touch, e.g. hidden_state)
//   MDN      mu = raw[0:n], std = safe_exp(raw[n:2n]), n = len/2
//            (parse_mdn with in_N = out_N = 0, parse_model_outputs.py:43-84)
//   SIGMOID  1 / (1 + safe_exp(-x))              (:8-9, parse_binary_crossentropy)
//   SOFTMAX  max-shifted softmax over groups of `width` consecutive values
//            (:11-18, parse_categorical_crossentropy)
//   MHP      in_N hypotheses of [mu(n) | std-logits(n) | out_N weight logits]:
//            weights = softmax over hypotheses per selection; for out_N == 1
//            the hypotheses are reordered by descending weight; selection h
//            takes the hypothesis np.argsort(w[:, h])[::-1][0] picks
//            (parse_model_outputs.py:50-75).
// safe_exp(x) = exp(min(x, 11)) (parse_model_outputs.py:4-6).
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

__device__ __forceinline__ float safe_exp(float x) { return expf(fminf(x, 11.0f)); }

constexpr int MHP_MAX_N = 8;

__global__ __launch_bounds__(256) void decode_kernel(const float* __restrict__ raw, float* __restrict__ dec,
                                                     const DecodeHead* __restrict__ heads, int n_heads,
                                                     unsigned* counter, const float* __restrict__ hn,
                                                     float* __restrict__ feat, int H) {
  if ((int)blockIdx.x == n_heads) {
    // end of frame (the last workgroup when a counter is given): advance the
    // queue frame counter and feed the new hidden state back into the packed
    // input's prev_feat slot (run_pinned2.py:1580 done on device).  Nothing
    // else in this launch reads either.
    if (threadIdx.x == 0) counter[0] = counter[0] + 1u;
    for (int j = threadIdx.x; j < H; j += 256) feat[j] = hn[j];
    return;
  }
  const DecodeHead h = heads[blockIdx.x];
  const float* in = raw + h.in_off;
  float* out = dec + h.out_off;
  const int t = threadIdx.x;
  switch (h.kind) {
    case DEC_RAW:
      for (int i = t; i < h.len; i += 256) out[i] = in[i];
      break;
    case DEC_MDN:
      for (int i = t; i < h.n; i += 256) {
        out[i] = in[i];
        out[h.n + i] = safe_exp(in[h.n + i]);
      }
      break;
    case DEC_SIGMOID:
      for (int i = t; i < h.len; i += 256) out[i] = 1.0f / (1.0f + safe_exp(-in[i]));
      break;
    case DEC_SOFTMAX:
      for (int g = t; g < h.len / h.width; g += 256) {
        const float* x = in + g * h.width;
        float* y = out + g * h.width;
        float mx = x[0];
        for (int i = 1; i < h.width; ++i) mx = fmaxf(mx, x[i]);
        float s = 0.f;
        for (int i = 0; i < h.width; ++i) {
          y[i] = safe_exp(x[i] - mx);
          s += y[i];
        }
        for (int i = 0; i < h.width; ++i) y[i] /= s;
      }
      break;
    case DEC_MHP: {
      // out: weights [in_N][out_N] | hyp mu [in_N][n] | hyp std [in_N][n] | mu [out_N][n] | std [out_N][n]
      const int N = h.in_N, S = h.out_N, n = h.n, L = 2 * n + S;
      float* w = out;
      float* hmu = w + N * S;
      float* hstd = hmu + N * n;
      float* fmu = hstd + N * n;
      float* fstd = fmu + S * n;
      __shared__ int order[MHP_MAX_N];
      __shared__ int pick[MHP_MAX_N];
      if (t == 0) {
        float wl[MHP_MAX_N][MHP_MAX_N];
        for (int j = 0; j < S; ++j) {
          float mx = in[0 * L + 2 * n + j];
          for (int i = 1; i < N; ++i) mx = fmaxf(mx, in[i * L + 2 * n + j]);
          float s = 0.f;
          for (int i = 0; i < N; ++i) {
            wl[i][j] = safe_exp(in[i * L + 2 * n + j] - mx);
            s += wl[i][j];
          }
          for (int i = 0; i < N; ++i) wl[i][j] /= s;
        }
        // hypothesis order: reversed stable ascending sort of w[:, 0] when
        // out_N == 1 (descending, equal weights by descending index), else identity
        for (int i = 0; i < N; ++i) order[i] = i;
        if (S == 1)
          for (int i = 1; i < N; ++i)
            for (int k = i; k > 0; --k) {
              const float a = wl[order[k - 1]][0], b = wl[order[k]][0];
              if (a < b || (a == b && order[k - 1] < order[k])) {
                const int tmp = order[k - 1];
                order[k - 1] = order[k];
                order[k] = tmp;
              } else {
                break;
              }
            }
        for (int i = 0; i < N; ++i)
          for (int j = 0; j < S; ++j) w[i * S + j] = wl[order[i]][j];
        // selection h: the last index among the maxima of the (reordered) w[:, h]
        for (int j = 0; j < S; ++j) {
          int best = 0;
          for (int i = 1; i < N; ++i)
            if (w[i * S + j] >= w[best * S + j]) best = i;
          pick[j] = order[best];
        }
      }
      __syncthreads();
      for (int e = t; e < N * n; e += 256) {
        const int i = e / n, k = e % n, src = order[i];
        hmu[e] = in[src * L + k];
        hstd[e] = safe_exp(in[src * L + n + k]);
      }
      for (int e = t; e < S * n; e += 256) {
        const int j = e / n, k = e % n, src = pick[j];
        fmu[e] = in[src * L + k];
        fstd[e] = safe_exp(in[src * L + n + k]);
      }
      break;
    }
    default:
      break;
  }
}

}  // namespace

void launch_decode(const float* raw, float* decoded, const DecodeHead* heads_dev, int n_heads, hipStream_t s,
                   unsigned* counter, const float* h, float* packed_feat, int H) {
  CK_REQUIRE(raw && decoded && heads_dev && n_heads > 0, "decode: bad arguments");
  CK_REQUIRE(!counter || (h && packed_feat && H > 0), "decode: the frame tick needs h, packed_feat and H");
  CK_LAUNCH(decode_kernel, dim3(n_heads + (counter ? 1 : 0)), dim3(256), 0, s, raw, decoded, heads_dev,
                     n_heads, counter, h, packed_feat, H);
  CK_LAUNCHED("decode");
}

}  // namespace ck
