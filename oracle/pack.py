"""Oracle restatements of uint8 frame packing and the policy input queues.

Test infrastructure only (see oracle/__init__.py).  All integer / copy work:
the device path must match these bit for bit.
"""
import numpy as np


def yuv_to_channels(Y, U, V):
    """Full-resolution Y, U, V planes (uint8 [H, W] each, H and W even) ->
    uint8 [6, H/2, W/2] = [Y00, Y10, Y01, Y11, U00, V00].

    Restates the tail of `rgb_to_channels` after cv2's resize and RGB->YUV
    conversion (video_check.py:27-32, identical in video_demo.py and
    drive_gui.py): Y[0::2,0::2], Y[1::2,0::2], Y[0::2,1::2], Y[1::2,1::2],
    U[0::2,0::2], V[0::2,0::2].  The cv2 steps before it are out of scope.
    Pinned by: brute-force per-pixel loop on a hand-built frame.
    """
    Y, U, V = (np.asarray(p, dtype=np.uint8) for p in (Y, U, V))
    return np.stack([Y[0::2, 0::2], Y[1::2, 0::2], Y[0::2, 1::2], Y[1::2, 1::2],
                     U[0::2, 0::2], V[0::2, 0::2]]).astype(np.uint8)


def frames_to_tensor(frames):
    """I420 frame uint8 [H*3/2, W] -> uint8 [6, H/2, W/2].

    Restates compile_modeld.py:83-92: the four Y phases by stride-2 slicing,
    then the U plane (rows H .. H+H/4) and the V plane (rows H+H/4 .. H+H/2)
    each reshaped to [H/2, W/2].
    Pinned by: brute-force loop on a hand-built frame whose bytes encode
    their own coordinates.
    """
    frames = np.asarray(frames, dtype=np.uint8)
    H = (frames.shape[0] * 2) // 3
    W = frames.shape[1]
    return np.concatenate([
        frames[0:H:2, 0::2][None],
        frames[1:H:2, 0::2][None],
        frames[0:H:2, 1::2][None],
        frames[1:H:2, 1::2][None],
        frames[H:H + H // 4].reshape((1, H // 2, W // 2)),
        frames[H + H // 4:H + H // 2].reshape((1, H // 2, W // 2)),
    ], axis=0)


# ---------------------------------------------------------------------------
# policy input queues (compile_modeld.py:121-221; run_pinned2.py:1372-1389)
# ---------------------------------------------------------------------------
FRAME_SKIP = 4          # run_pinned2.py:1373 (hard-coded there)
PACKED_LEN = 8 + 2 + 2 + 512   # desire8 | traffic_convention2 | action_t2 | prev_feat512


def shift_push(buf, new):
    """buf[1:] ++ new along axis 0 (compile_modeld.py:166-168)."""
    return np.concatenate([buf[1:], new[None]], axis=0)


def sample_skip(buf, fs=FRAME_SKIP):
    """buf[::fs] flattened over its first two axes (compile_modeld.py:171-172)."""
    s = buf[::fs]
    return s.reshape((s.shape[0] * s.shape[1],) + s.shape[2:])


def sample_desire(buf, fs=FRAME_SKIP):
    """max over consecutive groups of fs entries (compile_modeld.py:175-176)."""
    g = buf.reshape((-1, fs) + buf.shape[1:]).max(axis=1)
    return g.reshape((g.shape[0] * g.shape[1],) + g.shape[2:])


class PolicyQueues:
    """The four policy input queues with the reference's shapes and zero init.

    img_q / big_img_q: uint8 (FS*(n_frames-1)+1, 6, H, W) = (5, 6, 128, 256)
    feat_q: f32 (FS*24, 1, 512); desire_q: f32 (FS*25, 1, 8)
    (run_pinned2.py:1374-1384; compile_modeld.py:121-157).
    """

    def __init__(self, img_h=128, img_w=256, n_frames=2, feat_hist=24, feat_len=512,
                 desire_hist=25, desire_len=8, fs=FRAME_SKIP):
        self.fs = fs
        self.img_q = np.zeros((fs * (n_frames - 1) + 1, 6, img_h, img_w), np.uint8)
        self.big_img_q = np.zeros_like(self.img_q)
        self.feat_q = np.zeros((fs * feat_hist, 1, feat_len), np.float32)
        self.desire_q = np.zeros((fs * desire_hist, 1, desire_len), np.float32)
        self.desire_len = desire_len

    def step(self, warped, packed):
        """One `run_policy` input stage (compile_modeld.py:198-212).

        warped uint8 [2, 6, H, W]; packed f32 [desire | tc2 | action_t2 | prev_feat].
        Returns dict of img, big_img (uint8 [6*n_frames, H, W]), desire_pulse
        (f32 [25, 8]), features_buffer (f32 [24, 512]), traffic_convention (f32 [2]),
        action_t (f32 [2]).
        """
        warped = np.asarray(warped, np.uint8)
        packed = np.asarray(packed, np.float32)
        dl = self.desire_len
        desire = packed[0:dl]
        tc = packed[dl:dl + 2]
        at = packed[dl + 2:dl + 4]
        prev_feat = packed[dl + 4:]
        self.img_q = shift_push(self.img_q, warped[0])
        self.big_img_q = shift_push(self.big_img_q, warped[1])
        self.desire_q = shift_push(self.desire_q, desire.reshape(1, -1))
        self.feat_q = shift_push(self.feat_q, prev_feat.reshape(1, -1))
        return {
            'img': sample_skip(self.img_q, self.fs),
            'big_img': sample_skip(self.big_img_q, self.fs),
            'desire_pulse': sample_desire(self.desire_q, self.fs),
            'features_buffer': sample_skip(self.feat_q, self.fs),
            'traffic_convention': tc.copy(),
            'action_t': at.copy(),
        }
