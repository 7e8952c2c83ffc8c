"""Pinning the NV12 warp restatement (oracle/warp.py) with closed forms:
identity and integer translations are copies with edge clamping, a 2x
scale is subsampling, exact half coordinates round to even, the border-fill
branch masks exactly the out-of-range pixels, and the UV transform samples
the interleaved plane at half resolution."""
import numpy as np

from oracle import warp as W
from oracle import pack as OP


def _nv12(rng, w, h, stride, y_height):
    buf = rng.integers(0, 256, stride * y_height + (h // 2) * stride, dtype=np.uint8)
    return buf


def test_identity_is_a_copy():
    rng = np.random.default_rng(0)
    src = rng.integers(0, 256, 12 * 16, dtype=np.uint8)
    out = W.warp_perspective(src, np.eye(3), (16, 12), (12, 16), 0)
    np.testing.assert_array_equal(out, src)


def test_translation_clamps_to_edge_and_border_fill():
    src = np.arange(6 * 8, dtype=np.uint8)
    M = np.array([[1, 0, 3], [0, 1, -2], [0, 0, 1]], np.float32)      # src = (x + 3, y - 2)
    out = W.warp_perspective(src, M, (8, 6), (6, 8), 0).reshape(6, 8)
    img = src.reshape(6, 8)
    for y in range(6):
        for x in range(8):
            assert out[y, x] == img[min(max(y - 2, 0), 5), min(x + 3, 7)]
    fill = W.warp_perspective(src, M, (8, 6), (6, 8), 0, border_fill_val=255).reshape(6, 8)
    inside = np.zeros((6, 8), bool)
    inside[2:, :5] = True
    np.testing.assert_array_equal(fill[inside], out[inside])
    assert np.all(fill[~inside] == 255)


def test_scale_two_subsamples_and_stride_pad():
    rng = np.random.default_rng(1)
    h, w, pad = 10, 12, 4
    img = rng.integers(0, 256, (h, w + pad), dtype=np.uint8)
    out = W.warp_perspective(img.reshape(-1), np.diag([2.0, 2.0, 1.0]), (6, 5), (h, w), pad).reshape(5, 6)
    np.testing.assert_array_equal(out, img[0:10:2, 0:12:2])


def test_round_half_to_even():
    src = np.arange(8, dtype=np.uint8)
    M = np.array([[1, 0, 0.5], [0, 1, 0], [0, 0, 1]], np.float32)     # src_x = x + 0.5 exactly
    out = W.warp_perspective(src, M, (7, 1), (1, 8), 0)
    np.testing.assert_array_equal(out, [0, 2, 2, 4, 4, 6, 6])         # 0.5->0, 1.5->2, 2.5->2, ...


def test_projective_divide():
    src = np.arange(100, dtype=np.uint8)
    M = np.array([[2, 0, 0], [0, 2, 0], [0, 0, 2]], np.float32)       # homogeneous scale: identity
    np.testing.assert_array_equal(W.warp_perspective(src, M, (10, 10), (10, 10), 0), src)


def test_frame_prepare_identity_equals_frames_to_tensor():
    """With the identity transform and model size = camera size the warp is
    the plain NV12 -> 6-channel packing; it must agree with the I420 packing
    oracle on the deinterleaved planes."""
    rng = np.random.default_rng(2)
    w, h, stride, yh = 16, 8, 20, 10
    buf = _nv12(rng, w, h, stride, yh)
    out = W.frame_prepare(buf, np.eye(3, dtype=np.float32), w, h, stride, yh, h // 2, w, h)
    Y = buf[:h * stride].reshape(h, stride)[:, :w]
    UV = buf[stride * yh:stride * yh + (h // 2) * stride].reshape(h // 2, stride)
    i420 = np.concatenate([Y.reshape(-1), UV[:, 0:w:2].reshape(-1), UV[:, 1:w:2].reshape(-1)]).reshape(h * 3 // 2, w)
    np.testing.assert_array_equal(out, OP.frames_to_tensor(i420))
    assert out.shape == (6, h // 2, w // 2)
