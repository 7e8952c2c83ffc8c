"""Per-frame rows file and bit-identity gate (video_check.py:34-36, 47-94).

video_check.py runs a clip through run_frame with the hidden state fed back,
reduces every frame's plan to one row

    (frame index, speed ~1.75 s ahead, lateral offset at ~2 s, speed at ~2 s,
     steer = clip(lateral / 2, -1, 1))

of the plan hypothesis whose last point is closest to the lane centre
(plan viewed as 5 hypotheses x 33 points x 6, video_check.py:34-36), prints
a summary and saves the rows as .npy (video_check.py:94).  Rows files of two
runs are then compared bit for bit (graph replay vs eager, one build vs
another).  Here the frames come from a .npy of uint8 [N, 6, 128, 256]
channel frames or are generated from a seed (no video decoder is available);
the overlay video needs OpenCV and is not produced.

    python -m chestnut.rows run  --spec big_driving_1b --frames 60 --out rows.npy [--eager]
    python -m chestnut.rows gate rows_a.npy rows_b.npy
"""
import argparse
import sys

import numpy as np

LOOKAHEAD = 8   # plan point ~2 s ahead (video_check.py:62)
ROW_FIELDS = ('frame', 'v_now', 'lateral', 'v_next', 'steer')


def plan_row(out, out_slices, index, lookahead=LOOKAHEAD):
    """One rows-file row from a flat output vector (video_check.py:34-36, 62-66)."""
    plan = np.asarray(out[out_slices['plan']]).reshape(5, 33, 6)
    tr = plan[int(np.argmin(np.abs(plan[:, -1, 1])))]
    v_now = float(np.linalg.norm(tr[max(1, lookahead - 1), 3:6]))
    v_next = float(np.linalg.norm(tr[lookahead, 3:6]))
    steer = max(-1.0, min(1.0, float(tr[lookahead, 1]) / 2.0))
    return (index, v_now, float(tr[lookahead, 1]), v_next, steer)


def summary(rows):
    """The statistics video_check.py:89-93 prints."""
    r = np.asarray(rows, np.float64)
    return {'frames': int(len(r)),
            'v_next_mean': float(r[:, 3].mean()), 'v_next_min': float(r[:, 3].min()),
            'v_next_max': float(r[:, 3].max()),
            'steer_mean': float(r[:, 4].mean()), 'steer_min': float(r[:, 4].min()),
            'steer_max': float(r[:, 4].max()),
            'decel_frames': int((r[:, 3] < r[:, 1] * 0.9).sum()),
            'stop_frames': int((r[:, 3] < 1).sum())}


def run_rows(run_frame, out_slices, frames, packed=None):
    """Feed channel frames (uint8 [6,128,256] each) through run_frame with the
    hidden state fed back (video_check.py:47-66); both streams get the same
    frame, as video_check does.  Returns float64 rows [N, 5]."""
    pk = np.zeros(524, np.float32) if packed is None else np.array(packed, np.float32)
    if packed is None:
        pk[8:10] = (1.0, 0.0)
    rows = []
    for i, ch in enumerate(frames):
        ch = np.asarray(ch, np.uint8)
        out = run_frame(np.stack([ch, ch]), pk)
        pk[12:] = out[out_slices['hidden_state']]
        rows.append(plan_row(out, out_slices, i))
    return np.array(rows, np.float64).reshape(-1, len(ROW_FIELDS))


def gate(a, b):
    """Bit-identity of two rows arrays: (identical, first differing row or None)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.shape != b.shape:
        return False, -1
    diff = np.any(a.view(np.uint64) != b.view(np.uint64), axis=1)
    bad = np.flatnonzero(diff)
    return (len(bad) == 0), (int(bad[0]) if len(bad) else None)


def synthetic_frames(n, seed=0):
    """Seeded stand-in for a decoded clip: a slowly drifting random texture,
    so consecutive frames are correlated as video frames are."""
    rng = np.random.default_rng(seed)
    base = rng.integers(0, 256, (6, 128, 256)).astype(np.int16)
    for i in range(n):
        noise = rng.integers(-8, 9, base.shape)
        yield np.clip(np.roll(base, i, axis=2) + noise, 0, 255).astype(np.uint8)


def _main(argv=None):
    ap = argparse.ArgumentParser(prog='python -m chestnut.rows')
    sub = ap.add_subparsers(dest='cmd', required=True)
    r = sub.add_parser('run')
    r.add_argument('--spec', default='big_driving_1b')
    r.add_argument('--frames', type=int, default=60)
    r.add_argument('--input', default=None, help='.npy of uint8 [N, 6, 128, 256] channel frames')
    r.add_argument('--seed', type=int, default=0)
    r.add_argument('--eager', action='store_true', help='plain launches instead of graph replay (REPLAY=0)')
    r.add_argument('--out', default='rows.npy')
    g = sub.add_parser('gate')
    g.add_argument('a')
    g.add_argument('b')
    a = ap.parse_args(argv)
    if a.cmd == 'gate':
        ok, first = gate(np.load(a.a), np.load(a.b))
        print(f'bit-identical={ok}' + ('' if ok else f' first differing row={first}'))
        return 0 if ok else 1
    from .engine import Engine
    frames = np.load(a.input)[:a.frames] if a.input else synthetic_frames(a.frames, a.seed)
    with Engine(a.spec, graph=not a.eager) as eng:
        rows = run_rows(eng.run_frame, eng.out_slices, frames)
    np.save(a.out, rows)
    s = summary(rows)
    print(f"processed {s['frames']} frames -> {a.out}")
    print(f"planned speed@2s: mean={s['v_next_mean']:.1f} min={s['v_next_min']:.1f} max={s['v_next_max']:.1f} m/s")
    print(f"steer: mean={s['steer_mean']:+.3f} min={s['steer_min']:+.3f} max={s['steer_max']:+.3f}")
    print(f"decel frames (v@2s < v@prev-step*0.9): {s['decel_frames']}")
    print(f"stop frames (v@2s < 1): {s['stop_frames']}")
    return 0


if __name__ == '__main__':
    sys.exit(_main())
