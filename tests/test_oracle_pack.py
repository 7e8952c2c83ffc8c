"""Pins the oracle's packing, queue and image-addressing restatements (CPU)."""
import numpy as np

from conftest import golden
from oracle import image as I
from oracle import pack as P


def test_yuv_packing_golden():
    z = golden('pack_kat.npz')
    np.testing.assert_array_equal(P.yuv_to_channels(z['Y'], z['U'], z['V']), z['out'])


def test_frames_to_tensor_golden():
    z = golden('i420_kat.npz')
    np.testing.assert_array_equal(P.frames_to_tensor(z['frame']), z['out'])


def test_frames_to_tensor_full_size_shape():
    f = np.random.default_rng(0).integers(0, 256, (384, 512), dtype=np.uint8)
    out = P.frames_to_tensor(f)
    assert out.shape == (6, 128, 256) and out.dtype == np.uint8


def test_queues_golden():
    z = golden('queue_kat.npz')
    fs, n_img, feat_hist, feat_len, des_hist, des_len = (int(v) for v in z['shape'])
    q = P.PolicyQueues(img_h=2, img_w=3, n_frames=n_img, feat_hist=feat_hist, feat_len=feat_len,
                       desire_hist=des_hist, desire_len=des_len, fs=fs)
    for f in range(z['frames'].shape[0]):
        warped = np.stack([z['frames'][f], z['frames'][f][::-1].copy()])
        out = q.step(warped, z['packed'][f])
        np.testing.assert_array_equal(out['img'], z['img'][f])
        np.testing.assert_array_equal(out['features_buffer'], z['feat'][f])
        np.testing.assert_array_equal(out['desire_pulse'], z['desire'][f])
        np.testing.assert_array_equal(out['traffic_convention'], z['packed'][f][des_len:des_len + 2])
        np.testing.assert_array_equal(out['action_t'], z['packed'][f][des_len + 2:des_len + 4])


def test_queue_default_shapes():
    q = P.PolicyQueues()
    assert q.img_q.shape == (5, 6, 128, 256)
    assert q.feat_q.shape == (96, 1, 512)
    assert q.desire_q.shape == (100, 1, 8)
    out = q.step(np.zeros((2, 6, 128, 256), np.uint8), np.zeros(524, np.float32))
    assert out['img'].shape == (12, 128, 256)
    assert out['features_buffer'].shape == (24, 512)
    assert out['desire_pulse'].shape == (25, 8)


def test_sampler_kat_golden():
    z = golden('sampler_kat.json')
    img = np.array(z['data'], np.float32).reshape(z['height'], z['width'], z['lanes'])
    for c in z['cases']:
        np.testing.assert_array_equal(I.img_texel_zero_border(img, c['y'], c['x']), c['expect'])
        np.testing.assert_array_equal(I.gather(img, [[c['y'], c['x']]])[0], c['expect'])


def test_gather_matches_scalar_rule():
    rng = np.random.default_rng(1)
    img = rng.integers(0, 255, (5, 7, 4), dtype=np.uint8)
    yx = rng.integers(-3, 10, (200, 2))
    g = I.gather(img, yx)
    for (y, x), row in zip(yx, g):
        np.testing.assert_array_equal(row, I.img_texel_zero_border(img, y, x))


def test_edge_clamp_variant():
    img = np.arange(2 * 3 * 1).reshape(2, 3, 1)
    assert I.img_texel_edge_clamp(img, -5, -5)[0] == 0
    assert I.img_texel_edge_clamp(img, 9, 9)[0] == 5
    np.testing.assert_array_equal(I.gather(img, [[-1, 1], [1, 7]], mode='edge')[:, 0], [1, 5])
