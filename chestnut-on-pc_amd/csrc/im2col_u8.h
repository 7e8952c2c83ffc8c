// Conv-stem layer 1 im2col as a device function, shared by its own kernel
// (pack.hip) and by the launch that also carries the temporal GEMV
// (gemv.hip).  Patch row p = (ho, wo) of a 3x3 stride-2 pad-1 conv, column
// k = (ky*3 + kx)*C + c, zero-padded to Kp columns; the input is uint8 planes
// [batch][C][H][W], each plane an image of A=H rows of B=W one-byte texels
// read with a zero border, value (u8 - 128) / 128.  Thread i of batch b
// writes the 8 consecutive columns k0 = (i % (Kp/8)) * 8 .. +7 of patch row
// i / (Kp/8): one 16-byte store, and the (tap, channel) pair of each column
// advanced by increment instead of a division per element (32-bit index
// math; the host checks the sizes fit).
#pragma once

#include "common.h"

namespace ck {

// The 8 values of thread i of batch b and their byte offset in `patches`;
// false (nothing to store) past the end of the batch's patch matrix.
// plane(c): the first texel of input channel c of batch b.
template <class Plane>
__device__ __forceinline__ bool im2col_u8_gather_p(Plane plane, int C, int H, int W, int Kp, int Ho, int Wo, int b,
                                                   int i, half8_t& v, long& off) {
  const int kg = Kp / 8;
  const int per = Ho * Wo * kg;
  if (i >= per) return false;
  const int p = i / kg, k0 = (i - p * kg) * 8;
  const int ho = p / Wo, wo = p - ho * Wo;
  int tap = k0 / C, c = k0 - tap * C;
  // every load is unconditional and in bounds (padding columns past the 9
  // taps re-read tap 8 and are zeroed), so all eight issue before any wait
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int tp = min(tap, 8);
    const int y = 2 * ho - 1 + tp / 3, x = 2 * wo - 1 + tp % 3;
    const int fl = y * W + x;
    const int fc = min(max(fl, 0), H * W - 1);
    const bool valid = (tap < 9) & (x >= 0) & (x < W) & (y >= 0) & (y < H);
    const uint8_t u = plane(c)[fc];
    v[e] = (half_t)(valid ? ((float)u - 128.0f) * 0.0078125f : 0.f);
    if (++c == C) {
      c = 0;
      ++tap;
    }
  }
  off = 2L * (((long)b * Ho * Wo + p) * Kp + k0);
  return true;
}

// Planes [batch][C][H][W] in one buffer.
__device__ __forceinline__ bool im2col_u8_gather(const uint8_t* __restrict__ img, int C, int H, int W, int Kp, int Ho,
                                                 int Wo, int b, int i, half8_t& v, long& off) {
  const uint8_t* base = img + (long)b * C * H * W;
  const long hw = (long)H * W;
  return im2col_u8_gather_p([&](int c) { return base + c * hw; }, C, H, W, Kp, Ho, Wo, b, i, v, off);
}

__device__ __forceinline__ void im2col_u8_at(const uint8_t* __restrict__ img, int C, int H, int W,
                                             half_t* __restrict__ patches, int Kp, int Ho, int Wo, int batch, int b,
                                             int i) {
  half8_t v;
  long off;
  // device-scope store: the layer-1 conv GEMM reads the patches next
  if (im2col_u8_gather(img, C, H, W, Kp, Ho, Wo, b, i, v, off))
    store_sc1(sc1_rsrc(patches, 2L * batch * Ho * Wo * Kp), off, v);
}

}  // namespace ck
