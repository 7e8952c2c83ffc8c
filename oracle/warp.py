"""Oracle restatement of the NV12 perspective warp that produces `warped`
(compile_modeld.py:53-118, 181-193).  Test infrastructure only (see
oracle/__init__.py).

All coordinate arithmetic is float32, operation by operation as the
reference writes it (no fused multiply-add):
  src_x = (M00*x + M01*y) + M02, src_y likewise, src_w likewise,
  src_x /= src_w, src_y /= src_w  (div='ieee': the correctly rounded f32
  quotient; div='rcp': src_x * rcp(src_w) with the correctly rounded f32
  reciprocal, the form the reference's engine rewrites every f32 division
  into, run_pinned2.py:622-628 -- the two differ by at most an ulp or so,
  which can move a rounding at a .5 boundary by one texel),
  x_round = round(src_x) (half to even), clipped to [0, w_src-1], cast int,
  idx = y_clip * (w_src + stride_pad) + x_clip, sample = src[idx],
  optionally replaced by border_fill where the rounded coordinate is
  outside the source.
"""
import numpy as np

F = np.float32


DIVISIONS = ('ieee', 'rcp')


def warp_rounded(M_inv, dst_shape, div='ieee'):
    """The rounded source coordinates (x_round, y_round) of every destination
    pixel, row-major (compile_modeld.py:58-69)."""
    if div not in DIVISIONS:
        raise ValueError(f'div must be one of {DIVISIONS}')
    w_dst, h_dst = dst_shape
    M = np.asarray(M_inv, F)
    x = np.broadcast_to(np.arange(w_dst, dtype=F)[None, :], (h_dst, w_dst)).reshape(-1)
    y = np.broadcast_to(np.arange(h_dst, dtype=F)[:, None], (h_dst, w_dst)).reshape(-1)
    src_x = (M[0, 0] * x + M[0, 1] * y) + M[0, 2]
    src_y = (M[1, 0] * x + M[1, 1] * y) + M[1, 2]
    src_w = (M[2, 0] * x + M[2, 1] * y) + M[2, 2]
    if div == 'ieee':
        src_x = (src_x / src_w).astype(F)
        src_y = (src_y / src_w).astype(F)
    else:
        r = (F(1.0) / src_w).astype(F)
        src_x = (src_x * r).astype(F)
        src_y = (src_y * r).astype(F)
    return np.rint(src_x), np.rint(src_y)


def warp_perspective(src_flat, M_inv, dst_shape, src_shape, stride_pad, border_fill_val=None, div='ieee'):
    """warp_perspective_tinygrad (compile_modeld.py:53-79)."""
    h_src, w_src = src_shape
    x_round, y_round = warp_rounded(M_inv, dst_shape, div)
    x_c = np.clip(x_round, 0, w_src - 1).astype(np.int64)
    y_c = np.clip(y_round, 0, h_src - 1).astype(np.int64)
    idx = y_c * (w_src + stride_pad) + x_c
    sampled = np.asarray(src_flat)[idx]
    if border_fill_val is None:
        return sampled
    inb = (x_round >= 0) & (x_round <= w_src - 1) & (y_round >= 0) & (y_round <= h_src - 1)
    return np.where(inb, sampled, np.asarray(border_fill_val, sampled.dtype))


UV_SCALE = np.array([[1.0, 1.0, 0.5], [1.0, 1.0, 0.5], [2.0, 2.0, 1.0]], F)


def frame_prepare(frame, M_inv, cam_w, cam_h, stride, y_height, uv_height, model_w, model_h, div='ieee'):
    """frame_prepare_tinygrad (compile_modeld.py:97-117): NV12 frame (flat u8)
    -> 6-channel u8 [6, model_h/2, model_w/2] via frames_to_tensor."""
    frame = np.asarray(frame, np.uint8).reshape(-1)
    uv_offset = stride * y_height
    stride_pad = stride - cam_w
    M_inv = np.asarray(M_inv, F)
    M_inv_uv = (M_inv * UV_SCALE).astype(F)
    uv = frame[uv_offset:uv_offset + uv_height * stride].reshape(uv_height, stride)
    y = warp_perspective(frame[:cam_h * stride], M_inv, (model_w, model_h), (cam_h, cam_w), stride_pad, div=div)
    u = warp_perspective(uv[:cam_h // 2, :cam_w:2].reshape(-1), M_inv_uv, (model_w // 2, model_h // 2),
                         (cam_h // 2, cam_w // 2), 0, div=div)
    v = warp_perspective(uv[:cam_h // 2, 1:cam_w:2].reshape(-1), M_inv_uv, (model_w // 2, model_h // 2),
                         (cam_h // 2, cam_w // 2), 0, div=div)
    yuv = np.concatenate([y, u, v]).reshape(model_h * 3 // 2, model_w)
    H, W = model_h, model_w
    return np.stack([yuv[0:H:2, 0::2], yuv[1:H:2, 0::2], yuv[0:H:2, 1::2], yuv[1:H:2, 1::2],
                     yuv[H:H + H // 4].reshape(H // 2, W // 2), yuv[H + H // 4:H + H // 2].reshape(H // 2, W // 2)])


def warp(tfm, big_tfm, frame, big_frame, nv12, model_w, model_h, div='ieee'):
    """make_warp's warp (compile_modeld.py:181-193): both frames ->
    u8 [2, 6, model_h/2, model_w/2].  nv12 = (cam_w, cam_h, stride, y_height, uv_height)."""
    return np.stack([frame_prepare(frame, tfm, *nv12, model_w, model_h, div=div),
                     frame_prepare(big_frame, big_tfm, *nv12, model_w, model_h, div=div)])
