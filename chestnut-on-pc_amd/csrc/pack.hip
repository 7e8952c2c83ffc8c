// Integer-exact input-side kernels: policy input queues, uint8 frame packing,
// image2d zero-border gathers and the conv-stem im2col built on them.
#include "common.h"
#include "im2col_u8.h"
#include "kernels.h"
#include "policy_inputs.h"

namespace ck {
namespace {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

__global__ __launch_bounds__(256) void policy_inputs_kernel(const PolicyArgs a) {
  policy_inputs_at(a, (long)blockIdx.x * 256 + threadIdx.x);
}

// ---------------------------------------------------------------------------
// uint8 frame packing.
// ---------------------------------------------------------------------------
// [Y00, Y10, Y01, Y11, U00, V00] from full-resolution planes
// (video_check.py:27-32).  Thread per output pixel.
__global__ __launch_bounds__(256) void yuv_to_channels_kernel(const uint8_t* __restrict__ Y, const uint8_t* __restrict__ U,
                                                              const uint8_t* __restrict__ V, int H, int W,
                                                              uint8_t* __restrict__ out) {
  const int h2 = H / 2, w2 = W / 2;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)h2 * w2) return;
  const int r = (int)(i / w2), c = (int)(i % w2);
  const long plane = (long)h2 * w2;
  const long y0 = (long)(2 * r) * W + 2 * c, y1 = y0 + W;
  out[i] = Y[y0];
  out[plane + i] = Y[y1];
  out[2 * plane + i] = Y[y0 + 1];
  out[3 * plane + i] = Y[y1 + 1];
  out[4 * plane + i] = U[y0];
  out[5 * plane + i] = V[y0];
}

// frames_to_tensor (compile_modeld.py:83-92): I420 [H*3/2][W] -> [6][H/2][W/2].
// The U and V planes are contiguous runs of H/4 full rows, i.e. H*W/4 bytes
// each, read in order as [H/2][W/2].
__global__ __launch_bounds__(256) void i420_to_channels_kernel(const uint8_t* __restrict__ f, int H, int W,
                                                               uint8_t* __restrict__ out) {
  const int h2 = H / 2, w2 = W / 2;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)h2 * w2) return;
  const int r = (int)(i / w2), c = (int)(i % w2);
  const long plane = (long)h2 * w2;
  const long y0 = (long)(2 * r) * W + 2 * c, y1 = y0 + W;
  out[i] = f[y0];
  out[plane + i] = f[y1];
  out[2 * plane + i] = f[y0 + 1];
  out[3 * plane + i] = f[y1 + 1];
  out[4 * plane + i] = f[(long)H * W + i];
  out[5 * plane + i] = f[(long)H * W + plane + i];
}

// ---------------------------------------------------------------------------
// image2d zero-border gather (run_pinned2.py:56-84, 355-374).
// ---------------------------------------------------------------------------
template <typename TexelT>
__global__ __launch_bounds__(256) void img_gather_kernel(const TexelT* __restrict__ img, int A, int B,
                                                         const int* __restrict__ yx, int n, TexelT* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  out[i] = img_texel_zb(img, A, B, yx[2 * i], yx[2 * i + 1]);
}

template <int LANES, typename E>
struct alignas(sizeof(E) * LANES) Texel {
  E v[LANES];
};

template <typename TexelT>
void gather_launch(const void* img, int A, int B, const int* yx, int n, void* out, hipStream_t s) {
  CK_LAUNCH(img_gather_kernel<TexelT>, dim3(ceil_div(n, 256)), dim3(256), 0, s,
                     static_cast<const TexelT*>(img), A, B, yx, n, static_cast<TexelT*>(out));
  CK_LAUNCHED("img_gather");
}

// ---------------------------------------------------------------------------
// Conv-stem im2col.  Patch row p = (ho, wo) of a 3x3 stride-2 pad-1 conv,
// column k = (ky*3 + kx)*C + c, zero-padded to Kp columns.  Every input read
// is an image2d texel read with a zero border.
// ---------------------------------------------------------------------------
// Layer 1: uint8 planes [batch][C][H][W] (im2col_u8_at, im2col_u8.h).
__global__ __launch_bounds__(256) void im2col_u8_kernel(const uint8_t* __restrict__ img, int C, int H, int W,
                                                        half_t* __restrict__ patches, int Kp, int Ho, int Wo) {
  im2col_u8_at(img, C, H, W, patches, Kp, Ho, Wo, (int)gridDim.y, (int)blockIdx.y,
               (int)(blockIdx.x * 256 + threadIdx.x));
}

// Later layers: f16 activations [batch][H][W][C] = an image of A=H rows of
// B=W*C/4 texels of 4 halves.  Thread per 4-column texel of the patch row.
__global__ __launch_bounds__(256) void im2col_f16_kernel(const half_t* __restrict__ act, int C, int H, int W,
                                                         half_t* __restrict__ patches, int Kp, int Ho, int Wo) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int kq = Kp / 4;
  const int per = Ho * Wo * kq;
  const int b = blockIdx.y;
  if (i >= per) return;
  const int p = i / kq;
  const int k = (i - p * kq) * 4;
  u32x2_t v = {0u, 0u};
  if (k < 9 * C) {
    const int tap = k / C, c = k - tap * C;
    const int ho = p / Wo, wo = p - ho * Wo;
    const int y = 2 * ho - 1 + tap / 3, xs = 2 * wo - 1 + tap % 3;
    const int B = W * (C / 4);
    // texel column: xs = -1 gives x in [-C/4, 0), xs = W gives x >= B, so the
    // zero-border rule alone supplies the conv padding
    const int x = xs * (C / 4) + c / 4;
    const u32x2_t* im = reinterpret_cast<const u32x2_t*>(act + (long)b * H * W * C);
    v = img_texel_zb(im, H, B, y, x);
  }
  reinterpret_cast<u32x2_t*>(patches + (long)b * Ho * Wo * Kp)[i] = v;
}

// Channels-as-tokens: F[c][s*NS + p] = stem_out[s][p][c].
__global__ __launch_bounds__(256) void tokens_kernel(const half_t* __restrict__ so, int NS, int C5,
                                                     half_t* __restrict__ F) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= 2 * NS * C5) return;
  const int c = i / (2 * NS), j = i % (2 * NS);
  const int s = j / NS, p = j % NS;
  F[i] = so[((long)s * NS + p) * C5 + c];
}

}  // namespace

void launch_policy_inputs(const QueueDims& q, const uint8_t* warped, const float* packed, const unsigned* counter,
                          uint8_t* img_ring, float* feat_ring, float* desire_ring, uint8_t* img_out, float* feat_out,
                          float* ctx_tail, hipStream_t s) {
  const PolicyArgs a =
      make_policy_args(q, warped, packed, counter, img_ring, feat_ring, desire_ring, img_out, feat_out, ctx_tail);
  CK_LAUNCH(policy_inputs_kernel, dim3(ceil_div(policy_inputs_threads(a), 256)), dim3(256), 0, s, a);
  CK_LAUNCHED("policy_inputs");
}

void launch_yuv_to_channels(const uint8_t* Y, const uint8_t* U, const uint8_t* V, int H, int W, uint8_t* out,
                            hipStream_t s) {
  CK_REQUIRE(Y && U && V && out, "yuv_to_channels: null pointer");
  CK_REQUIRE(H > 0 && W > 0 && H % 2 == 0 && W % 2 == 0, "yuv_to_channels: H and W must be positive and even");
  CK_LAUNCH(yuv_to_channels_kernel, dim3(ceil_div((long)(H / 2) * (W / 2), 256)), dim3(256), 0, s, Y, U, V,
                     H, W, out);
  CK_LAUNCHED("yuv_to_channels");
}

void launch_i420_to_channels(const uint8_t* frame, int H, int W, uint8_t* out, hipStream_t s) {
  CK_REQUIRE(frame && out, "i420_to_channels: null pointer");
  CK_REQUIRE(H > 0 && W > 0 && H % 4 == 0 && W % 2 == 0, "i420_to_channels: H must be a multiple of 4, W even");
  CK_LAUNCH(i420_to_channels_kernel, dim3(ceil_div((long)(H / 2) * (W / 2), 256)), dim3(256), 0, s, frame,
                     H, W, out);
  CK_LAUNCHED("i420_to_channels");
}

void launch_img_gather(const void* img, int A, int B, int lanes, int elem_bytes, const int* yx, int n, void* out,
                       hipStream_t s) {
  CK_REQUIRE(img && yx && out, "img_gather: null pointer");
  CK_REQUIRE(A > 0 && B > 0 && (long)A * B < (1L << 31), "img_gather: bad image size");
  if (n <= 0) return;
  const int tb = lanes * elem_bytes;
  CK_REQUIRE((reinterpret_cast<uintptr_t>(img) % tb) == 0 && (reinterpret_cast<uintptr_t>(out) % tb) == 0,
             "img_gather: image and output must be aligned to the texel size");
  switch (tb) {
    case 1: gather_launch<Texel<1, uint8_t>>(img, A, B, yx, n, out, s); break;
    case 2: gather_launch<Texel<1, uint16_t>>(img, A, B, yx, n, out, s); break;
    case 4: gather_launch<Texel<1, uint32_t>>(img, A, B, yx, n, out, s); break;
    case 8: gather_launch<Texel<2, uint32_t>>(img, A, B, yx, n, out, s); break;
    case 16: gather_launch<Texel<4, uint32_t>>(img, A, B, yx, n, out, s); break;
    default: throw Error("img_gather: texel size must be 1, 2, 4, 8 or 16 bytes");
  }
}

void launch_im2col_u8(const uint8_t* img, int batch, int C, int H, int W, half_t* patches, int Kp, hipStream_t s) {
  CK_REQUIRE(img && patches && batch > 0, "im2col_u8: bad arguments");
  CK_REQUIRE(Kp >= 9 * C && Kp % 8 == 0, "im2col_u8: Kp must be >= 9C and a multiple of 8");
  CK_REQUIRE((reinterpret_cast<uintptr_t>(patches) & 15) == 0, "im2col_u8: patches must be 16-byte aligned");
  const int Ho = (H - 1) / 2 + 1, Wo = (W - 1) / 2 + 1;
  const long per = (long)Ho * Wo * (Kp / 8);
  CK_REQUIRE(per < (1L << 31) && (long)H * W < (1L << 31), "im2col_u8: image too large");
  // the patches leave through raw buffer stores addressed by 32-bit offsets
  CK_REQUIRE(2L * batch * Ho * Wo * Kp < (1L << 31), "im2col_u8: patch buffer must be under 2 GiB");
  CK_LAUNCH(im2col_u8_kernel, dim3(ceil_div(per, 256), batch), dim3(256), 0, s, img, C, H, W, patches, Kp,
                     Ho, Wo);
  CK_LAUNCHED("im2col_u8");
}

void launch_im2col_f16(const half_t* act, int batch, int C, int H, int W, half_t* patches, int Kp, hipStream_t s) {
  CK_REQUIRE(act && patches && batch > 0, "im2col_f16: bad arguments");
  CK_REQUIRE(C % 4 == 0 && Kp % 4 == 0 && Kp >= 9 * C, "im2col_f16: C and Kp must be multiples of 4, Kp >= 9C");
  const int Ho = (H - 1) / 2 + 1, Wo = (W - 1) / 2 + 1;
  const long per = (long)Ho * Wo * (Kp / 4);
  CK_REQUIRE(per < (1L << 31), "im2col_f16: image too large");
  CK_LAUNCH(im2col_f16_kernel, dim3(ceil_div(per, 256), batch), dim3(256), 0, s, act, C, H, W, patches, Kp,
                     Ho, Wo);
  CK_LAUNCHED("im2col_f16");
}

void launch_tokens(const half_t* stem_out, int n_spatial, int C5, half_t* F, hipStream_t s) {
  CK_LAUNCH(tokens_kernel, dim3(ceil_div(2L * n_spatial * C5, 256)), dim3(256), 0, s, stem_out, n_spatial,
                     C5, F);
  CK_LAUNCHED("tokens");
}

}  // namespace ck
