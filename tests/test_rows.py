"""Rows file and gate of chestnut.rows (video_check.py:34-36, 47-94), host logic."""
import numpy as np

from chestnut import rows as R
from chestnut import spec as S


def _out_with_plan(plan):
    sl = S.output_slices('tiny')
    out = np.zeros(sl['hidden_state'].stop, np.float32)
    out[sl['plan']] = np.asarray(plan, np.float32).reshape(-1)
    return out, sl


def test_plan_row_closed_form():
    plan = np.zeros((5, 33, 6), np.float32)
    plan[:, -1, 1] = [3.0, -2.0, 0.5, -0.25, 1.0]       # hypothesis 3 ends closest to the centre
    plan[3, 7, 3:6] = (3.0, 4.0, 0.0)                     # |v| = 5 at point 7
    plan[3, 8, 3:6] = (6.0, 8.0, 0.0)                     # |v| = 10 at point 8
    plan[3, 8, 1] = 0.6
    plan[0, 8, 3:6] = (100.0, 0.0, 0.0)                   # other hypotheses are ignored
    out, sl = _out_with_plan(plan)
    assert R.plan_row(out, sl, 7) == (7, 5.0, np.float32(0.6), 10.0, np.float32(0.6) / 2.0)
    plan[3, 8, 1] = -5.0                                  # steer clips at -1
    out, sl = _out_with_plan(plan)
    assert R.plan_row(out, sl, 0)[4] == -1.0


def test_summary_counts():
    rows = np.array([[0, 10.0, 0.0, 8.0, 0.1],     # decel (8 < 9)
                     [1, 10.0, 0.0, 9.5, -0.3],
                     [2, 1.0, 0.0, 0.5, 0.2]])     # decel and stop
    s = R.summary(rows)
    assert s['decel_frames'] == 2 and s['stop_frames'] == 1 and s['frames'] == 3
    assert s['v_next_max'] == 9.5 and s['steer_min'] == -0.3


def test_gate_bit_identity():
    a = np.arange(15, dtype=np.float64).reshape(3, 5)
    assert R.gate(a, a.copy()) == (True, None)
    b = a.copy()
    b[2, 4] = np.nextafter(b[2, 4], 100)                 # one ulp
    assert R.gate(a, b) == (False, 2)
    z = a.copy()
    z[1, 1] = -0.0
    y = a.copy()
    y[1, 1] = 0.0
    assert R.gate(z, y) == (False, 1)                    # bits, not values
    assert R.gate(a, a[:2]) == (False, -1)


def test_run_rows_recurrence_with_stub():
    """The hidden state of frame i is frame i+1's packed[12:] (video_check.py:60)."""
    sl = S.output_slices('tiny')
    seen = []

    def run_frame(warped, pk):
        assert warped.shape == (2, 6, 128, 256) and np.array_equal(warped[0], warped[1])
        seen.append(pk[12:].copy())
        out = np.zeros(sl['hidden_state'].stop, np.float32)
        out[sl['hidden_state']] = len(seen)
        return out

    rows = R.run_rows(run_frame, sl, R.synthetic_frames(3, seed=1))
    assert rows.shape == (3, 5) and list(rows[:, 0]) == [0, 1, 2]
    assert [float(h[0]) for h in seen] == [0.0, 1.0, 2.0]
