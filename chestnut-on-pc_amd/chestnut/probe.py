"""Per-kernel probe and A/B bench of one frame-plan entry.

The reference studies one kernel at a time in two steps: a probe runs a
real frame and dumps the kernel's pre-state buffers (r62_probe.py:1-80,
alu_probe.py:1-60), then a bench replays that kernel on a fresh context
15 times, baseline and variant, and prints median / min time plus
bit-identical / ndiff / maxabs / maxrel of the variant's output against the
baseline's (bench_r62.py:25-65).  Here:

  capture   run `frames` frames of make_warped(val) (the last one only up to
            the entry), snapshot the whole frame state (every non-parameter
            tensor, including the split-K workspace), run the entry once and
            snapshot again; then time the entry `reps` times, each launch on
            a restored pre-state, between HIP events on the engine stream.
            Writes DIR/meta.json, DIR/pre.npz, DIR/post.npz.

  bench     rebuild the same engine (same spec and seeded weights) with a
            variant -- another build of the library (--lib, the analogue of
            the reference's variant cubin) and/or a GEMM tile/split for this
            entry (--gemm TILE,SPLIT, the analogue of its local-size
            argument) -- restore the captured pre-state, time the entry the
            same way and compare every state tensor with post.npz.

  fingerprint  run `warm` frames of make_warped(val) through the graph or
            plain launches, then `frames` eager frames launch by launch: each
            launch's pre-state fingerprint (a device hash of every state
            tensor, ck_state_hashes) and its time, printed as KSYNC prints
            them (run_pinned2.py:1519-1550) and written to a JSON file.

  diff      two fingerprint files (graph against eager warm frames, one
            build against another, one spec option against another): the
            first launch after which the states differ, and the tensors that
            differ there -- xcheck's launch-by-launch comparison of two runs
            (research/xcheck.py:65-124, 150-200).

    python -m chestnut.probe capture --spec big_driving_1b --entry blk0.up --out DIR
    python -m chestnut.probe bench DIR [--lib PATH] [--gemm 5,2] [--reps 15] [--ignore ws]
    python -m chestnut.probe fingerprint --spec tiny [--warm 3 --warm-mode graph] [--lib PATH] --out A.json
    python -m chestnut.probe diff A.json B.json [--ignore ws]

Timings are per launch (HIP events around the single entry, no host
launch overhead), so `med` is the kernel's own duration.
"""
import argparse
import hashlib
import json
import os
import sys

import numpy as np


def _engine(spec, lib=None):
    if lib:
        from . import _lib
        _lib.LIB_PATH = os.path.abspath(lib)
    from .engine import Engine
    from . import spec as S
    return Engine(spec, weights=S.make_weights(spec))


def _time_entry(eng, idx, pre, reps):
    ts = []
    for _ in range(reps):
        eng.restore(pre)
        ts.append(eng.time_launches([idx], 1))
    return ts


def compare(base, var, ignore=()):
    """bench_r62.py:57-65 statistics over every state tensor: bit-identical,
    number of differing elements, max abs / max rel difference over the
    floating-point elements where the baseline is non-zero.  `per_tensor`
    holds (ndiff, maxabs, maxrel) of each differing tensor; tensors named in
    `ignore` (scratch such as the split-K workspace "ws", which variants
    with another split fill differently) are listed there but left out of
    the totals."""
    ndiff, maxabs, maxrel = 0, 0.0, 0.0
    changed = []
    per = {}
    for name, b in base.items():
        v = var[name]
        if b.shape != v.shape or b.dtype != v.dtype:
            raise ValueError(f'{name}: shape/dtype differ ({b.shape} {b.dtype} vs {v.shape} {v.dtype})')
        diff = b.view(np.uint8).reshape(-1, b.itemsize) != v.view(np.uint8).reshape(-1, b.itemsize)
        nd = int(diff.any(axis=1).sum())
        if not nd:
            continue
        ma, mr = 0.0, 0.0
        if b.dtype.kind == 'f':
            b64, v64 = b.astype(np.float64), v.astype(np.float64)
            nz = b64 != 0
            if nz.any():
                d = np.abs(b64[nz] - v64[nz])
                ma = float(np.nanmax(d))
                mr = float(np.nanmax(d / np.maximum(1e-30, np.abs(b64[nz]))))
        per[name] = (nd, ma, mr)
        if name in ignore:
            continue
        changed.append(name)
        ndiff += nd
        maxabs, maxrel = max(maxabs, ma), max(maxrel, mr)
    return {'bit_identical': ndiff == 0, 'ndiff': ndiff, 'maxabs': maxabs, 'maxrel': maxrel, 'changed': changed,
            'per_tensor': per}


def fmt_times(ts):
    s = sorted(ts)
    return f'med={s[len(s) // 2]:.4f}ms min={s[0]:.4f}ms'


def capture(spec_name, entry, out, frames=1, val=111, reps=15, gemm=None):
    from . import spec as S
    sp = S.get_spec(spec_name)
    if gemm:
        sp = dict(sp, gemm_config={entry: list(gemm)})
    eng = _engine(sp)
    names = [e['name'] for e in eng.plan()]
    if entry not in names:
        raise SystemExit(f'unknown plan entry {entry!r}; entries: {", ".join(names)}')
    idx = names.index(entry)
    plan = eng.plan()[idx]
    warped = eng.make_warped(val)
    packed = eng.PACKED.copy()
    packed[8:10] = (1.0, 0.0)
    for _ in range(frames - 1):
        o = eng.run_frame(warped, packed)
        packed[12:] = o[eng.out_slices['hidden_state']]
    eng.write('warped', warped)
    eng.write('packed', packed)
    eng.run_range(0, idx)
    pre = eng.snapshot()
    eng.run_range(idx, idx + 1)
    post = eng.snapshot()
    ts = _time_entry(eng, idx, pre, reps)
    eng.close()
    os.makedirs(out, exist_ok=True)
    np.savez(os.path.join(out, 'pre.npz'), **pre)
    np.savez(os.path.join(out, 'post.npz'), **post)
    meta = {'spec': sp, 'entry': entry, 'index': idx, 'kernel': plan['kernel'], 'flops': plan['flops'],
            'bytes': plan['bytes'], 'frames': frames, 'val': val, 'reps': reps, 'baseline_ms': ts,
            'state': {k: [str(v.dtype), int(v.size)] for k, v in pre.items()}}
    with open(os.path.join(out, 'meta.json'), 'w') as fh:
        json.dump(meta, fh, indent=1)
    return meta


def bench(d, lib=None, gemm=None, reps=None, ignore=()):
    meta = json.load(open(os.path.join(d, 'meta.json')))
    sp = dict(meta['spec'])
    if gemm:
        sp['gemm_config'] = dict(sp.get('gemm_config', {}), **{meta['entry']: list(gemm)})
    pre = dict(np.load(os.path.join(d, 'pre.npz')))
    base = dict(np.load(os.path.join(d, 'post.npz')))
    eng = _engine(sp, lib)
    idx = [e['name'] for e in eng.plan()].index(meta['entry'])
    if idx != meta['index']:
        raise SystemExit('the variant plan differs from the captured one')
    # a variant split-K factor resizes the workspace: restore its captured
    # prefix, and leave tensors whose size changed out of the comparison
    sizes = {n: nb // np.dtype(dt).itemsize for n, nb, dt in eng.state_names()}
    resized = [n for n, a in pre.items() if sizes[n] != a.size]
    for n in resized:
        a = np.zeros(sizes[n], pre[n].dtype)
        k = min(a.size, pre[n].size)
        a[:k] = pre[n][:k]
        pre[n] = a
        del base[n]
    eng.restore(pre)
    eng.run_range(idx, idx + 1)
    var = eng.snapshot()
    ts = _time_entry(eng, idx, pre, reps or meta['reps'])
    eng.close()
    res = compare(base, {n: var[n] for n in base}, ignore)
    res['resized'] = resized
    res['variant_ms'] = ts
    res['baseline_ms'] = meta['baseline_ms']
    return res


def state_digest(pre, ignore=()):
    """8 hex digits over a launch's whole pre-state (KSYNC's pre=...)."""
    h = hashlib.md5()
    for name in sorted(pre):
        if name not in ignore:
            h.update(f'{name}:{pre[name]:016x};'.encode())
    return h.hexdigest()[:8]


def fingerprint(spec, out=None, frames=1, warm=0, warm_mode='graph', val=111, lib=None, extra=None, log=print):
    """Fingerprinted eager frames after `warm` frames in `warm_mode`; returns
    (and writes to `out`) {'meta': ..., 'rows': Engine.fingerprints rows}."""
    from . import spec as S
    sp = dict(S.get_spec(spec), **(extra or {}))
    eng = _engine(sp, lib)
    try:
        warped = eng.make_warped(val)
        packed = eng.PACKED.copy()
        packed[8:10] = (1.0, 0.0)
        eng.set_graph(warm_mode == 'graph')
        for _ in range(warm):
            o = eng.run_frame(warped, packed)
            packed[12:] = o[eng.out_slices['hidden_state']]
        eng.write('warped', warped)
        eng.write('packed', packed)
        rows = eng.fingerprints(frames)
    finally:
        eng.close()
    for r in rows:
        ms = f"{r['ms']:7.3f}ms" if r['ms'] is not None else ' ' * 9
        log(f"[ksync] {r['frame']}:{r['index']:3d} {r['name']:32} {ms} pre={state_digest(r['pre'])}")
    tot = sum(r['ms'] for r in rows if r['ms'] is not None)
    log(f'[ksync] total kernel GPU time = {tot:.2f}ms over {sum(r["ms"] is not None for r in rows)} launches')
    res = {'meta': {'spec': sp['name'], 'frames': frames, 'warm': warm, 'warm_mode': warm_mode, 'val': val,
                    'lib': lib}, 'rows': [dict(r, pre={k: f'{v:016x}' for k, v in r['pre'].items()}) for r in rows]}
    if out:
        os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
        with open(out, 'w') as fh:
            json.dump(res, fh)
    return res


def diff(a, b, ignore=()):
    """First divergence of two fingerprint runs: rows are matched by (frame,
    index); at the first row whose pre-states differ, the launch before it
    (the previous row) is the first one whose results differ -- or, at row 0,
    the runs already differed before the fingerprinted frames.  Returns None
    when every pre-state agrees."""
    ra, rb = a['rows'], b['rows']
    if [(r['frame'], r['index'], r['name']) for r in ra] != [(r['frame'], r['index'], r['name']) for r in rb]:
        raise ValueError('the two runs have different plans or frame counts')
    for k, (x, y) in enumerate(zip(ra, rb)):
        dt = sorted(n for n in x['pre'] if n not in ignore and x['pre'][n] != y['pre'].get(n))
        if dt:
            prev = ra[k - 1] if k else None
            return {'row': k, 'before': x['name'], 'frame': x['frame'], 'index': x['index'],
                    'launch': (prev['name'] if prev else None), 'launch_index': (prev['index'] if prev else None),
                    'tensors': dt}
    return None


def main(argv=None):
    ap = argparse.ArgumentParser(prog='python -m chestnut.probe', description=__doc__.split('\n\n')[0])
    sub = ap.add_subparsers(dest='cmd', required=True)
    c = sub.add_parser('capture')
    c.add_argument('--spec', default='big_driving_1b')
    c.add_argument('--entry', required=True)
    c.add_argument('--out', required=True)
    c.add_argument('--frames', type=int, default=1)
    c.add_argument('--val', type=int, default=111)
    c.add_argument('--reps', type=int, default=15)
    c.add_argument('--gemm', default=None, help='TILE,SPLIT for the entry in the baseline')
    b = sub.add_parser('bench')
    b.add_argument('dir')
    b.add_argument('--lib', default=None)
    b.add_argument('--gemm', default=None, help='TILE,SPLIT for the entry in the variant')
    b.add_argument('--reps', type=int, default=None)
    b.add_argument('--ignore', default='', help='comma-separated scratch tensors left out of the totals (e.g. ws)')
    f = sub.add_parser('fingerprint')
    f.add_argument('--spec', default='big_driving_1b')
    f.add_argument('--out', required=True)
    f.add_argument('--frames', type=int, default=1)
    f.add_argument('--warm', type=int, default=0, help='frames run before the fingerprinted ones')
    f.add_argument('--warm-mode', choices=('graph', 'eager'), default='graph')
    f.add_argument('--val', type=int, default=111)
    f.add_argument('--lib', default=None)
    f.add_argument('--set', default=None, help='JSON object of spec options, e.g. {"fuse_head": 0}')
    d = sub.add_parser('diff')
    d.add_argument('a')
    d.add_argument('b')
    d.add_argument('--ignore', default='', help='comma-separated tensors left out (e.g. ws)')
    a = ap.parse_args(argv)
    if a.cmd == 'fingerprint':
        fingerprint(a.spec, a.out, a.frames, a.warm, a.warm_mode, a.val, a.lib,
                    json.loads(a.set) if a.set else None)
        return 0
    if a.cmd == 'diff':
        with open(a.a) as fa, open(a.b) as fb:
            r = diff(json.load(fa), json.load(fb), tuple(x for x in a.ignore.split(',') if x))
        if r is None:
            print('[diff] identical: every launch of both runs saw the same pre-state', flush=True)
            return 0
        if r['launch'] is None:
            print(f"[diff] the runs differ before the first fingerprinted launch ({r['before']}): "
                  f"{', '.join(r['tensors'])}", flush=True)
        else:
            print(f"[diff] first divergent launch: frame {r['frame']} #{r['launch_index']} {r['launch']} "
                  f"-> differs in {', '.join(r['tensors'])}", flush=True)
        return 1
    gemm = tuple(int(x) for x in a.gemm.split(',')) if a.gemm else None
    if a.cmd == 'capture':
        m = capture(a.spec, a.entry, a.out, a.frames, a.val, a.reps, gemm)
        print(f"[probe] {m['entry']} (plan index {m['index']}, {m['kernel']}): {len(m['state'])} state tensors "
              f"captured to {a.out}", flush=True)
        print(f"baseline: {fmt_times(m['baseline_ms'])}", flush=True)
    else:
        r = bench(a.dir, a.lib, gemm, a.reps, tuple(x for x in a.ignore.split(',') if x))
        print(f"baseline: {fmt_times(r['baseline_ms'])}")
        print(f"variant : {fmt_times(r['variant_ms'])}  bit-identical={r['bit_identical']} ndiff={r['ndiff']} "
              f"maxabs={r['maxabs']:.3e} maxrel={r['maxrel']:.3e}", flush=True)
        for name, (nd, ma, mr) in r['per_tensor'].items():
            print(f"          {name}: ndiff={nd} maxabs={ma:.3e} maxrel={mr:.3e}"
                  f"{' (ignored)' if name not in r['changed'] else ''}", flush=True)
        if r['resized']:
            print(f"          not compared (size differs in the variant): {', '.join(r['resized'])}", flush=True)


if __name__ == '__main__':
    sys.exit(main())
