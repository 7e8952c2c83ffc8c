"""CPU replay of the device queue rings (csrc/pack.hip policy_inputs_kernel).

The kernel keeps each policy queue as a ring indexed by a frame counter n and
reads frame n's own entry from the input staging.  This replay follows its
index arithmetic line by line on small shapes, for frame_skip 1, 2 and 4,
checks the sampled inputs against the reference's shift/sample queues
(oracle.pack.PolicyQueues, compile_modeld.py:166-212), and checks that no
ring read in a launch touches the slot the same launch writes (that would be
a race between workgroups)."""
import numpy as np
import pytest

from oracle import pack as OP


def wrap(f, n):
    return f % n


class RingReplay:
    def __init__(self, H, W, fs, feat_len, feat_hist, desire_len, desire_hist, n_frames=2):
        self.fs, self.fl, self.fh, self.dl, self.dh = fs, feat_len, feat_hist, desire_len, desire_hist
        self.slots = fs * (n_frames - 1) + 1
        self.img_ring = np.zeros((2, self.slots, 6, H, W), np.uint8)
        self.feat_ring = np.zeros((fs * feat_hist, feat_len), np.float32)
        self.desire_ring = np.zeros((fs * desire_hist, desire_len), np.float32)
        self.n = 0

    def launch(self, warped, packed):
        n, fs = self.n, self.fs
        dl = self.dl
        prev_feat = packed[dl + 4:]
        reads = {'img': set(), 'feat': set(), 'desire': set()}
        # image branch: frames n - (slots-1) from the ring and n from staging
        old_slot = wrap(n - (self.slots - 1), self.slots)
        reads['img'].add(old_slot)
        img = np.stack([np.concatenate([self.img_ring[s, old_slot], warped[s]]) for s in range(2)])
        # feature samples: k = 0..feat_hist-1
        fL = fs * self.fh
        feat = np.empty((self.fh, self.fl), np.float32)
        for k in range(self.fh):
            f = n - (fL - 1) + fs * k
            if f == n:
                feat[k] = prev_feat
            else:
                reads['feat'].add(wrap(f, fL))
                feat[k] = self.feat_ring[wrap(f, fL)]
        # desire group maxima
        dL = fs * self.dh
        des = np.empty((self.dh, dl), np.float32)
        for g in range(self.dh):
            for c in range(dl):
                m = 0.0
                for t in range(fs):
                    j = g * fs + t
                    f = n - (dL - 1) + j
                    if j == dL - 1:
                        v = packed[c]
                    else:
                        reads['desire'].add(wrap(f, dL))
                        v = self.desire_ring[wrap(f, dL), c]
                    m = v if (t == 0 or v > m) else m
                des[g, c] = m
        # the launch's writes: slot n of every ring
        writes = {'img': wrap(n, self.slots), 'feat': wrap(n, fL), 'desire': wrap(n, dL)}
        for q in reads:
            assert writes[q] not in reads[q], f'{q}: a read of ring slot {writes[q]} races with its push'
        for s in range(2):
            self.img_ring[s, writes['img']] = warped[s]
        self.feat_ring[writes['feat']] = prev_feat
        self.desire_ring[writes['desire']] = packed[:dl]
        self.n += 1      # the end-of-frame tick
        return img, feat, des, packed[dl:dl + 2], packed[dl + 2:dl + 4]


@pytest.mark.parametrize('fs', [1, 2, 3, 4])
def test_ring_replay_matches_reference_queues(fs):
    H, W, fl, fh, dl, dh = 4, 8, 3, 5, 8, 6
    rng = np.random.default_rng(100 + fs)
    rep = RingReplay(H, W, fs, fl, fh, dl, dh)
    ref = OP.PolicyQueues(img_h=H, img_w=W, feat_hist=fh, feat_len=fl, desire_hist=dh, desire_len=dl, fs=fs)
    for f in range(3 * fs * max(fh, dh) + 3):
        warped = rng.integers(0, 256, (2, 6, H, W), dtype=np.uint8)
        packed = np.concatenate([(rng.random(dl) > 0.6).astype(np.float32), rng.standard_normal(4 + fl)
                                 .astype(np.float32)])
        img, feat, des, tc, at = rep.launch(warped, packed)
        r = ref.step(warped, packed)
        np.testing.assert_array_equal(img[0], r['img'], err_msg=f'fs={fs} frame {f}')
        np.testing.assert_array_equal(img[1], r['big_img'])
        np.testing.assert_array_equal(feat, r['features_buffer'], err_msg=f'fs={fs} frame {f} feat')
        np.testing.assert_array_equal(des, r['desire_pulse'], err_msg=f'fs={fs} frame {f} desire')
        np.testing.assert_array_equal(tc, r['traffic_convention'])
        np.testing.assert_array_equal(at, r['action_t'])


def test_ring_replay_without_staging_read_races_for_fs1():
    """The form before the fix (the last feature sample read from the ring
    for frame_skip 1) reads the slot its own launch pushes."""
    fs, fh = 1, 4
    fL = fs * fh
    n = 7
    slots = {wrap(n - (fL - 1) + fs * k, fL) for k in range(fh)}
    assert wrap(n, fL) in slots


@pytest.mark.parametrize('fs', [1, 4])
def test_queues_view_unrolls_rings_to_reference_order(fs):
    """chestnut.engine.Queues rebuilds the reference's queue tensors from the
    rings and the frame counter; on the replayed rings it gives exactly
    PolicyQueues' img_q / big_img_q / feat_q / desire_q after every frame."""
    from chestnut.engine import Queues
    H, W, fl, fh, dl, dh = 4, 8, 3, 5, 8, 6
    rng = np.random.default_rng(200 + fs)
    rep = RingReplay(H, W, fs, fl, fh, dl, dh)
    ref = OP.PolicyQueues(img_h=H, img_w=W, feat_hist=fh, feat_len=fl, desire_hist=dh, desire_len=dl, fs=fs)
    for f in range(fs * dh + 5):
        warped = rng.integers(0, 256, (2, 6, H, W), dtype=np.uint8)
        packed = rng.standard_normal(dl + 4 + fl).astype(np.float32)
        rep.launch(warped, packed)
        ref.step(warped, packed)
        np.testing.assert_array_equal(Queues._unroll(rep.img_ring[0], rep.n), ref.img_q)
        np.testing.assert_array_equal(Queues._unroll(rep.img_ring[1], rep.n), ref.big_img_q)
        np.testing.assert_array_equal(Queues._unroll(rep.feat_ring[:, None], rep.n), ref.feat_q)
        np.testing.assert_array_equal(Queues._unroll(rep.desire_ring[:, None], rep.n), ref.desire_q)
