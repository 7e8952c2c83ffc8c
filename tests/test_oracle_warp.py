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


def _road_tfms(n, seed=0):
    """Seeded perturbations of a road-camera transform (model pixel ->
    camera pixel: scale about 3.7, offset into the frame, slight perspective)."""
    base = np.array([[3.7, -0.05, 10.0], [0.05, 3.7, 120.0], [1e-5, 2e-5, 1.0]], np.float32)
    rng = np.random.default_rng(seed)
    return [(base * (1 + 0.02 * rng.standard_normal((3, 3)))).astype(np.float32) for _ in range(n)]


def test_division_forms_differ_by_at_most_one_texel():
    """The reference writes src_x / src_w (compile_modeld.py:65-66); its engine
    lowers f32 divisions to x * rcp(y) (run_pinned2.py:622-628).  Counted over
    the Y and UV planes of 8 road-camera warps (1928x1208 -> 512x256): the two
    forms pick different texels at a handful of pixels per plane (35 of
    1,310,720 here), never more than one texel apart, and agree exactly
    wherever the transform is affine (src_w = 1)."""
    diff, total = 0, 0
    for M in _road_tfms(8):
        for Mx, dst in ((M, (512, 256)), ((M * W.UV_SCALE).astype(np.float32), (256, 128))):
            xi, yi = W.warp_rounded(Mx, dst, 'ieee')
            xr, yr = W.warp_rounded(Mx, dst, 'rcp')
            d = (xi != xr) | (yi != yr)
            diff += int(d.sum())
            total += d.size
            assert np.abs(xi - xr).max() <= 1 and np.abs(yi - yr).max() <= 1
    assert 0 < diff < 1e-4 * total, diff
    assert diff == 35
    affine = np.array([[3.7, -0.05, 10.25], [0.05, 3.7, 120.5], [0.0, 0.0, 1.0]], np.float32)
    for div in W.DIVISIONS:
        assert all(np.array_equal(a, b) for a, b in zip(W.warp_rounded(affine, (512, 256), 'ieee'),
                                                        W.warp_rounded(affine, (512, 256), div)))


def test_rcp_form_by_hand():
    """src_x * (1 / src_w) evaluated as two correctly rounded f32 operations:
    a case where it differs from the quotient, checked with exact rationals."""
    from fractions import Fraction as Fr
    F = np.float32
    # scan a small range for a pair whose two f32 forms disagree, then check both against exact arithmetic
    for sx_i in range(1, 4000):
        sx, sw = F(sx_i * 0.37), F(3.0)
        q, r = F(sx / sw), F(sx * F(F(1.0) / sw))
        if q != r:
            break
    else:
        raise AssertionError('no differing pair found')
    exact_q = Fr(float(sx)) / Fr(float(sw))
    exact_r = Fr(float(sx)) * Fr(float(F(F(1.0) / sw)))
    # each form is the f32 nearest its exact value
    for got, ex in ((q, exact_q), (r, exact_r)):
        nb = [np.nextafter(got, F(-np.inf)), got, np.nextafter(got, F(np.inf))]
        errs = [abs(Fr(float(v)) - ex) for v in nb]
        assert errs[1] == min(errs)
