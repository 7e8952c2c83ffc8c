"""Long recurrent clips (video_check.py:47-66): the hidden state fed back
frame after frame, the device and the oracle each running its own
recurrence, so element-level differences that grow over a clip would show
(NOTES.md:139-144: element-level noise moved frame-level plans in the
reference).  Every output slice of every frame stays within 1e-3 relative of
the f64 oracle; the video_check rows of graph replay and plain launches are
bit-identical over the same clip."""
import numpy as np
import pytest

from chestnut import Engine
from chestnut import rows as R
from chestnut import spec as S
from oracle import model as OM

pytestmark = pytest.mark.gpu
REL = 1e-3


def rel_err(got, ref):
    return float(np.max(np.abs(got.astype(np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def clip_inputs(spec, n, seed):
    """A drifting synthetic clip (correlated frames), desire pulses and
    action_t varying frame to frame, the traffic convention fixed."""
    s = S.get_spec(spec)
    rng = np.random.default_rng(seed)
    frames = list(R.synthetic_frames(n + 1, seed))
    for i in range(n):
        warped = np.stack([frames[i], frames[i + 1]])
        desire = np.zeros(s['desire_len'], np.float32)
        if i % 9 == 3:
            desire[rng.integers(0, s['desire_len'])] = 1.0
        extra = np.array([1.0, 0.0, *rng.uniform(-1, 1, 2)], np.float32)
        yield warped, desire, extra


def _clip(spec_name, n, seed, acc):
    sp = S.get_spec(spec_name)
    w = S.make_weights(sp)
    orc = OM.OracleModel(sp, w, acc=acc)
    worst = {}
    with Engine(sp, weights=w) as eng:
        pk_dev = np.zeros(524, np.float32)
        pk_ref = np.zeros(524, np.float32)
        for f, (warped, desire, extra) in enumerate(clip_inputs(sp, n, seed)):
            for pk in (pk_dev, pk_ref):
                pk[:8], pk[8:12] = desire, extra
            out = eng.run_frame(warped, pk_dev)
            ref = orc.run_frame(warped, pk_ref)
            errs = {name: rel_err(out[sl], ref[sl]) for name, sl in eng.out_slices.items()}
            print(f'[{spec_name}] frame {f:2d} ' + ' '.join(f'{k}={v:.1e}' for k, v in errs.items()), flush=True)
            for k, v in errs.items():
                worst[k] = max(worst.get(k, 0.0), v)
                assert v <= REL, (spec_name, f, k, v)
            pk_dev[12:] = out[eng.out_slices['hidden_state']]
            pk_ref[12:] = ref[eng.out_slices['hidden_state']]
    return worst


def test_tiny_40_frame_clip_vs_oracle(gpu):
    worst = _clip('tiny', 40, 5, np.float64)
    print(f'[tiny] worst over 40 frames {worst}', flush=True)


def test_39m_32_frame_clip_vs_oracle(gpu):
    worst = _clip('driving_39m', 32, 6, np.float64)
    print(f'[39m] worst over 32 frames {worst}', flush=True)


@pytest.mark.parametrize('spec_name,n', [('tiny', 40), ('driving_39m', 32)])
def test_rows_gate_graph_vs_eager_long_clip(gpu, spec_name, n):
    sp = S.get_spec(spec_name)
    frames = list(R.synthetic_frames(n, seed=9))
    with Engine(sp) as eng:
        a = R.run_rows(eng.run_frame, eng.out_slices, frames)
        eng.set_graph(False)
        eng.reset()
        b = R.run_rows(eng.run_frame, eng.out_slices, frames)
    ok, first = R.gate(a, b)
    print(f'[{spec_name}] rows graph vs eager over {n} frames: bit-identical={ok}', flush=True)
    assert ok, f'first differing row {first}'
