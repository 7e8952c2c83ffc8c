// NV12 perspective warp into the 6-channel model input: the gfx950 form of
// openpilot's frame_prepare (compile_modeld.py:53-118) for both frames of a
// step (make_warp, compile_modeld.py:181-193), fused with frames_to_tensor.
//
// For every destination pixel (x, y) of the model_w x model_h image:
//   src = M_inv . (x, y, 1), src_x /= src_w, src_y /= src_w   (f32)
//   xr, yr = round half to even; sample the source at the clipped (xr, yr)
// Y samples the full-resolution plane with M_inv; U and V sample the
// interleaved UV plane at half resolution with M_inv scaled by
// [[1,1,.5],[1,1,.5],[2,2,1]] (UV_SCALE . M_inv . UV_SCALE^-1).
// One thread owns output position (i, j) of the [model_h/2][model_w/2]
// channel planes: the four Y pixels (2i+{0,1}, 2j+{0,1}) -> channels 0..3
// (even/odd rows x even/odd columns) and U, V at (i, j) -> channels 4, 5.
//
// The coordinate arithmetic is f32 operation by operation with contraction
// off -- (M00*x + M01*y) + M02, then the division -- and the texel is the one
// that f32 arithmetic, evaluated in that order, selects.  The reference
// writes the division as src_x / src_w (compile_modeld.py:65-66); what that
// rounds to depends on how its graph is lowered (the reference's own engine
// rewrites every f32 division as x * rcp(y), run_pinned2.py:622-628), and
// the two forms pick different texels at a few .5 boundaries per frame.
// `rcp` selects the form: 0 the correctly rounded quotient, 1 the product
// with the correctly rounded reciprocal.
#include "common.h"
#include "kernels.h"

namespace ck {
namespace {

#pragma clang fp contract(off)
template <bool RCP>
__device__ __forceinline__ void warp_coord(const float* __restrict__ M, float x, float y, int w_src, int h_src, int& xc,
                                           int& yc) {
  const float sx = (M[0] * x + M[1] * y) + M[2];
  const float sy = (M[3] * x + M[4] * y) + M[5];
  const float sw = (M[6] * x + M[7] * y) + M[8];
  float qx, qy;
  if (RCP) {
    const float r = 1.0f / sw;   // correctly rounded (no fast-math reciprocal)
    qx = sx * r;
    qy = sy * r;
  } else {
    qx = sx / sw;
    qy = sy / sw;
  }
  const float xr = rintf(qx), yr = rintf(qy);
  xc = (int)fminf(fmaxf(xr, 0.f), (float)(w_src - 1));
  yc = (int)fminf(fmaxf(yr, 0.f), (float)(h_src - 1));
}
#pragma clang fp contract(on)

template <bool RCP>
__global__ __launch_bounds__(256) void warp_nv12_kernel(const uint8_t* __restrict__ f0, const uint8_t* __restrict__ f1,
                                                        const float* __restrict__ m0, const float* __restrict__ m1,
                                                        int cam_w, int cam_h, int stride, long uv_offset, int W, int H,
                                                        uint8_t* __restrict__ out) {
  const int Wh = W / 2, Hh = H / 2;
  const long n = (long)Hh * Wh;
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= 2 * n) return;
  const int f = (int)(t / n);
  const int p = (int)(t - (long)f * n);
  const int i = p / Wh, j = p % Wh;
  const uint8_t* src = f ? f1 : f0;
  const float* Mg = f ? m1 : m0;
  float M[9], Mu[9];
#pragma unroll
  for (int k = 0; k < 9; ++k) M[k] = Mg[k];
  // UV transform: columns 0,1 of rows 0,1 kept, (0,2),(1,2) halved, row 2's first two doubled
  Mu[0] = M[0]; Mu[1] = M[1]; Mu[2] = M[2] * 0.5f;
  Mu[3] = M[3]; Mu[4] = M[4]; Mu[5] = M[5] * 0.5f;
  Mu[6] = M[6] * 2.0f; Mu[7] = M[7] * 2.0f; Mu[8] = M[8];
  uint8_t* o = out + (long)f * 6 * n + p;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int yy = 2 * i + (c & 1), xx = 2 * j + (c >> 1);
    int xc, yc;
    warp_coord<RCP>(M, (float)xx, (float)yy, cam_w, cam_h, xc, yc);
    o[(long)c * n] = src[(long)yc * stride + xc];
  }
  int xc, yc;
  warp_coord<RCP>(Mu, (float)j, (float)i, cam_w / 2, cam_h / 2, xc, yc);
  const uint8_t* uv = src + uv_offset + (long)yc * stride + 2 * xc;
  o[4 * n] = uv[0];
  o[5 * n] = uv[1];
}

}  // namespace

void launch_warp_nv12(const uint8_t* frame, const uint8_t* big_frame, size_t frame_bytes, const float* tfm,
                      const float* big_tfm, int cam_w, int cam_h, int stride, int y_height, int model_w, int model_h,
                      int division, uint8_t* out, hipStream_t s) {
  CK_REQUIRE(frame && big_frame && tfm && big_tfm && out, "warp_nv12: null pointer");
  CK_REQUIRE(division == 0 || division == 1, "warp_nv12: division must be 0 (quotient) or 1 (reciprocal product)");
  CK_REQUIRE(cam_w > 0 && cam_h > 0 && cam_w % 2 == 0 && cam_h % 2 == 0, "warp_nv12: camera size must be even");
  CK_REQUIRE(stride >= cam_w && y_height >= cam_h, "warp_nv12: stride >= width and y_height >= height required");
  CK_REQUIRE(model_w > 0 && model_h > 0 && model_w % 4 == 0 && model_h % 4 == 0,
             "warp_nv12: model size must be a multiple of 4");
  const long uv_offset = (long)stride * y_height;
  CK_REQUIRE((size_t)(uv_offset + (long)(cam_h / 2) * stride) <= frame_bytes,
             "warp_nv12: frame buffer smaller than its Y plane and the UV rows the warp reads");
  const long n = 2L * (model_h / 2) * (model_w / 2);
  if (division)
    CK_LAUNCH(warp_nv12_kernel<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, frame, big_frame, tfm,
              big_tfm, cam_w, cam_h, stride, uv_offset, model_w, model_h, out);
  else
    CK_LAUNCH(warp_nv12_kernel<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, frame, big_frame, tfm,
              big_tfm, cam_w, cam_h, stride, uv_offset, model_w, model_h, out);
  CK_LAUNCHED("warp_nv12");
}

}  // namespace ck
