"""NV12 perspective warp on the GPU against the oracle, bit for bit
(compile_modeld.py:53-118 restated in oracle/warp.py)."""
import numpy as np
import pytest

from oracle import warp as OW

pytestmark = pytest.mark.gpu

CAM = dict(cam_w=1928, cam_h=1208, stride=2048, y_height=1216)   # a road-camera-sized NV12 frame


def _frame(rng):
    n = CAM['stride'] * CAM['y_height'] + (CAM['cam_h'] // 2) * CAM['stride']
    return rng.integers(0, 256, n, dtype=np.uint8)


def _tfms(rng):
    # model (512x256) pixel -> camera pixel: scale ~3.7, offset to the middle, small
    # rotation and perspective; one that maps far outside the frame; one with exact
    # half-pixel coordinates (round half to even); the identity.
    a = 0.02 * rng.standard_normal()
    persp = np.array([[3.7 * np.cos(a), -3.7 * np.sin(a), 10.0], [3.7 * np.sin(a), 3.7 * np.cos(a), 120.0],
                      [1e-5 * rng.standard_normal(), 2e-5 * rng.standard_normal(), 1.0]], np.float32)
    far = np.array([[6.0, 0.3, -900.0], [-0.2, 5.5, -400.0], [0.0, 0.0, 1.0]], np.float32)
    half = np.array([[2.0, 0.0, 0.5], [0.0, 2.0, 1.5], [0.0, 0.0, 1.0]], np.float32)
    return [(persp, far), (half, np.eye(3, dtype=np.float32))]


@pytest.mark.parametrize('division', OW.DIVISIONS)
def test_warp_nv12_bit_exact(gpu, division):
    from chestnut import kernels as K
    torch = gpu
    rng = np.random.default_rng(7)
    frame, big = _frame(rng), _frame(rng)
    nv12 = (CAM['cam_w'], CAM['cam_h'], CAM['stride'], CAM['y_height'], CAM['cam_h'] // 2)
    for tfm, big_tfm in _tfms(rng):
        print(f'[warp] {division} tfm {tfm.ravel()[:3]} big {big_tfm.ravel()[:3]}', flush=True)
        got = K.warp_nv12(torch.from_numpy(frame).cuda(), torch.from_numpy(big).cuda(),
                          torch.from_numpy(tfm).cuda(), torch.from_numpy(big_tfm).cuda(), **CAM,
                          division=division).cpu().numpy()
        ref = OW.warp(tfm, big_tfm, frame, big, nv12, 512, 256, div=division)
        np.testing.assert_array_equal(got, ref)


def test_warp_nv12_division_forms(gpu):
    """Over seeded road-camera transforms the two division forms pick
    different texels at a few pixels; the device matches the oracle's form
    bit for bit in both, so the switch selects exactly the stated arithmetic."""
    from chestnut import kernels as K
    torch = gpu
    rng = np.random.default_rng(8)
    frame, big = _frame(rng), _frame(rng)
    nv12 = (CAM['cam_w'], CAM['cam_h'], CAM['stride'], CAM['y_height'], CAM['cam_h'] // 2)
    base = np.array([[3.7, -0.05, 10.0], [0.05, 3.7, 120.0], [1e-5, 2e-5, 1.0]], np.float32)
    differ = 0
    for t in range(4):
        tfm = (base * (1 + 0.02 * rng.standard_normal((3, 3)))).astype(np.float32)
        big_tfm = (base * (1 + 0.02 * rng.standard_normal((3, 3)))).astype(np.float32)
        print(f'[warp] forms transform {t}', flush=True)
        got = {}
        for div in OW.DIVISIONS:
            got[div] = K.warp_nv12(torch.from_numpy(frame).cuda(), torch.from_numpy(big).cuda(),
                                   torch.from_numpy(tfm).cuda(), torch.from_numpy(big_tfm).cuda(), **CAM,
                                   division=div).cpu().numpy()
            np.testing.assert_array_equal(got[div], OW.warp(tfm, big_tfm, frame, big, nv12, 512, 256, div=div))
        differ += int((got['ieee'] != got['rcp']).sum())
    assert differ > 0


def test_warp_nv12_rejects_short_buffer(gpu):
    from chestnut import kernels as K
    torch = gpu
    import ctypes
    from chestnut._lib import call
    f = torch.zeros(1000, dtype=torch.uint8, device='cuda')
    m = torch.eye(3, device='cuda')
    out = torch.empty(2, 6, 128, 256, dtype=torch.uint8, device='cuda')
    with pytest.raises(ValueError, match='must hold'):        # the torch harness, before any launch
        K.warp_nv12(f, f, m, m, **CAM)
    p = lambda t: ctypes.c_void_p(t.data_ptr())              # noqa: E731
    with pytest.raises(RuntimeError, match='frame buffer smaller'):   # the native entry point's own check
        call('ck_warp_nv12', p(f), p(f), f.numel(), p(m), p(m), CAM['cam_w'], CAM['cam_h'], CAM['stride'],
             CAM['y_height'], 512, 256, 0, p(out), None)
