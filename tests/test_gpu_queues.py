"""The drop-in namespace's `queues` (run_pinned2.py:1379-1386) rebuilt from
the device rings equals the reference's shift-by-one queues
(oracle.pack.PolicyQueues, compile_modeld.py:121-212) bit for bit, for the
default frame_skip 4 and for frame_skip 1 and 3 (where the last feature
sample is the current frame's own prev_feat)."""
import numpy as np
import pytest

from chestnut import engine as E
from chestnut import spec as S
from oracle import pack as OP

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('fs', [4, 1, 3])
def test_queues_view_and_sampled_inputs_match_reference(gpu, fs):
    sp = dict(S.get_spec('tiny'), frame_skip=fs)
    print(f'[queues] frame_skip={fs}', flush=True)
    ns = E.load(sp)
    eng = ns.engine
    try:
        assert set(ns.queues) == {'img_q', 'big_img_q', 'feat_q', 'desire_q', 'packed_npy_inputs'}
        ref = OP.PolicyQueues(fs=fs)
        for k in ('img_q', 'big_img_q', 'feat_q', 'desire_q'):
            np.testing.assert_array_equal(ns.queues[k], getattr(ref, k))        # zero-initialised
        rng = np.random.default_rng(fs)
        Td = sp['temporal_dim']
        n_frames = fs * 25 + 10          # past the longest ring (desire: fs * 25 entries)
        for f in range(n_frames):
            warped = rng.integers(0, 256, (2, 6, 128, 256), dtype=np.uint8)
            packed = np.zeros(524, np.float32)
            packed[:8] = (rng.random(8) > 0.7).astype(np.float32)
            packed[8:12] = rng.uniform(0, 1, 4).astype(np.float32)
            packed[12:] = rng.standard_normal(512).astype(np.float32)
            ns.run_frame(warped, packed)
            r = ref.step(warped, packed)
            np.testing.assert_array_equal(eng.read('feat_buf', np.float32, (24, 512)), r['features_buffer'],
                                          err_msg=f'fs={fs} frame {f} features')
            tail = eng.read('ctx_in', np.float32)[Td:Td + 204]
            np.testing.assert_array_equal(tail[:200].reshape(25, 8), r['desire_pulse'])
            img = eng.read('img', np.uint8, (2, 12, 128, 256))
            np.testing.assert_array_equal(img[0], r['img'])
            np.testing.assert_array_equal(img[1], r['big_img'])
            if f % 7 == 0 or f >= n_frames - 3:
                assert ns.queues.frames() == f + 1
                for k in ('img_q', 'big_img_q', 'feat_q', 'desire_q'):
                    np.testing.assert_array_equal(ns.queues[k], getattr(ref, k), err_msg=f'fs={fs} frame {f} {k}')
                np.testing.assert_array_equal(ns.queues['packed_npy_inputs'], packed)
        eng.reset()
        assert ns.queues.frames() == 0
        assert not ns.queues['feat_q'].any() and not ns.queues['img_q'].any()
    finally:
        eng.close()
