"""CPU replay of the implicit-convolution A addressing of gemm.hip
(conv_a_src and the per-lane row setup of gemm_dma_kernel with CV): for a
3x3 stride-2 pad-1 conv over an f16 [H][W][C] activation, the 16-byte chunk
that A row m (output pixel), columns k..k+7 gathers must equal the im2col
patch matrix [Ho*Wo][round_up(9C, 64)] (tap-major, channel-minor, zero
border and zero K padding) that the explicit path builds, and every chunk
read must lie inside the activation.  No GPU."""
import numpy as np
import pytest


def im2col(act):
    H, W, C = act.shape
    Ho, Wo = (H - 1) // 2 + 1, (W - 1) // 2 + 1
    Kp = -(-9 * C // 64) * 64
    pad = np.zeros((H + 2, W + 2, C), act.dtype)
    pad[1:-1, 1:-1] = act
    out = np.zeros((Ho * Wo, Kp), act.dtype)
    for dy in range(3):
        for dx in range(3):
            tap = dy * 3 + dx
            out[:, tap * C:(tap + 1) * C] = pad[dy:dy + 2 * Ho:2, dx:dx + 2 * Wo:2].reshape(Ho * Wo, C)
    return out


def gathered(act, M, Kp):
    """The kernel's view: row m -> (yb, xb) = (2*ho - 1, 2*wo - 1); chunk k ->
    tap = k >> log2(C), channel k & (C-1), dy = (tap*11) >> 5; out-of-image
    taps and tap >= 9 read the zero chunk."""
    H, W, C = act.shape
    cl = C.bit_length() - 1
    cwo = (W - 1) // 2 + 1
    flat = act.reshape(-1)
    out = np.empty((M, Kp), act.dtype)
    for m in range(M):
        ho, wo = m // cwo, m - (m // cwo) * cwo
        yb, xb = 2 * ho - 1, 2 * wo - 1
        for k in range(0, Kp, 8):
            tap, c = k >> cl, k & (C - 1)
            dy = (tap * 11) >> 5
            y, x = yb + dy, xb + tap - 3 * dy
            if tap < 9 and 0 <= y < H and 0 <= x < W:
                off = ((y * W + x) << cl) + c
                assert 0 <= off and off + 8 <= flat.size
                out[m, k:k + 8] = flat[off:off + 8]
            else:
                out[m, k:k + 8] = 0
    return out


def test_tap_division():
    assert [(t * 11) >> 5 for t in range(9)] == [t // 3 for t in range(9)]


@pytest.mark.parametrize('H,W,C', [(64, 128, 8), (32, 64, 16), (16, 32, 32), (8, 16, 64), (5, 7, 8), (9, 3, 256)])
def test_gather_equals_im2col(H, W, C):
    rng = np.random.default_rng(H * 1000 + W + C)
    act = rng.integers(1, 1 << 15, (H, W, C)).astype(np.int32)
    ref = im2col(act)
    assert (gathered(act, ref.shape[0], ref.shape[1]) == ref).all()
