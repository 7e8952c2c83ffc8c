"""Whole-frame tuning of the block GEMMs' tile and split.

A GEMM's time inside the frame differs from its time in a loop of launches
of its own family (measured on the 1B model: the per-family loop preferred
two K-groups for QKV and a 256x128 split-8 tile for MLP-down, both of which
lose on whole frames).  This tool therefore times whole frames: for each
block GEMM family in turn it builds the engine with every candidate
(tile, split) applied to all layers through the spec's `gemm_config`, times
back-to-back graph launches, and keeps the fastest (coordinate descent, the
families in order).  The result is a `gemm_config` object for the spec.

    python -m chestnut.tune --spec big_driving_1b [--families qkv,o,up,down,stem0,...,embed] [--frames 100]
                            [--out cfg.json]

The reference tunes its kernels with per-kernel variant benches (bench_r62.py,
bench_alu.py; the `probe` module here mirrors those); this is the frame-level
step on top of them.
"""
import argparse
import json
import sys
import time

import numpy as np

from . import spec as _spec

FAMILIES = ('qkv', 'o', 'up', 'down')        # per-block GEMMs (every layer gets the choice)
SINGLE = ('stem0', 'stem1', 'stem2', 'stem3', 'stem4', 'embed')   # once-per-frame GEMMs
# tile code -> (rows, columns) of the output tile (the codes of ck_gemm)
TILES = {1: (128, 128), 2: (128, 64), 3: (64, 128), 4: (64, 64), 5: (128, 128), 6: (128, 64), 7: (64, 128),
         8: (64, 64), 9: (256, 128), 10: (128, 96), 15: (32, 64)}


def shapes(sp):
    """family -> (M, N, K, epilogue kind, batch).  Kinds: 'frag' (QKV fragment
    epilogue, split 1), 'partials' (split-K partials read by the next LN),
    'f16' (fused activation, split 1), 'conv' (implicit-conv stem layer:
    split allowed, LDS-DMA tiles 1-8 only), 'reduce' (split allowed, summed
    by the split-K reduce kernel)."""
    T, d, F = sp['stem'][-1], sp['d_model'], sp['d_ff']
    out = {'qkv': (T, 3 * d, d, 'frag', 1), 'o': (T, d, d, 'partials', 1), 'up': (T, F, d, 'f16', 1),
           'down': (T, d, F, 'partials', 1)}
    H, W, C = sp['img_h'], sp['img_w'], 6 * sp['n_frames']
    for i, co in enumerate(sp['stem']):
        H, W = (H - 1) // 2 + 1, (W - 1) // 2 + 1
        # layers after the first run as implicit-conv GEMMs (LDS-DMA tiles 1-8)
        out[f'stem{i}'] = (H * W, co, -(-9 * C // 64) * 64, 'reduce' if i == 0 else 'conv', 2)
        C = co
    n_spatial = (sp['img_h'] >> len(sp['stem'])) * (sp['img_w'] >> len(sp['stem']))
    out['embed'] = (T, d, 2 * n_spatial, 'reduce', 1)
    return out


def entry_names(sp, fam):
    """Plan entries a family's choice applies to."""
    if fam in FAMILIES:
        return [f'blk{i}.{fam}' for i in range(sp['n_layers'])]
    return [f'{fam}.conv'] if fam.startswith('stem') else [fam]


def candidates(M, N, K, kind, batch=1, min_wg=64, max_wg=1024):
    """(tile, split) pairs the engine accepts for this GEMM: splits up to 16
    that give every split two or more 64-wide K-steps, split only where the
    epilogue allows it (the QKV fragment and fused-activation epilogues need
    split 1), the fragment epilogue only on tiles whose N divides, and a grid
    of min_wg..max_wg workgroups (fewer when the GEMM cannot fill min_wg)."""
    out = []
    for t, (bm, bn) in TILES.items():
        if kind == 'frag' and (N % bn or M % 32):
            continue
        if t == 9 and kind in ('frag', 'conv'):
            continue
        if t == 10 and kind != 'frag':   # the 128x96 tile serves the QKV fragment epilogue only
            continue
        for s in range(1, 17):
            if s > 1 and kind not in ('partials', 'reduce', 'conv'):
                continue
            if kind == 'partials' and s > 8:   # the residual LayerNorm sums at most 8 partials
                continue
            if K % (64 * s) or (s > 1 and K // (64 * s) < 2):
                continue
            grid = -(-M // bm) * -(-N // bn) * s * batch
            if min(min_wg, -(-M // 64) * -(-N // 64) * batch) <= grid <= max_wg:
                out.append((t, s))
    return out


def config_for(sp, choice):
    cfg = {}
    for fam, (t, s) in choice.items():
        for name in entry_names(sp, fam):
            cfg[name] = [t, s]
    return cfg


def time_frames(sp, weights, frames=100, warmup=10, names=None):
    """ms per frame of back-to-back graph launches; `names`, a list, receives
    the names of the plan's GEMM entries."""
    from .engine import Engine
    with Engine(sp, weights=weights) as eng:
        if names is not None:
            names.extend(e['name'] for e in eng.plan() if e['kernel'].startswith('gemm'))
        rng = np.random.default_rng(42)
        w = rng.integers(0, 256, (2, 6, sp['img_h'], sp['img_w']), dtype=np.uint8)
        p = np.zeros(sp['desire_len'] + 4 + sp['feat_len'], np.float32)
        p[8:10] = (1.0, 0.0)
        eng.run_frame(w, p)
        for _ in range(warmup):
            eng.frame_launch()
        eng.synchronize()
        t0 = time.perf_counter()
        for _ in range(frames):
            eng.frame_launch()
        eng.synchronize()
        return (time.perf_counter() - t0) * 1e3 / frames


def tune(spec='big_driving_1b', families=FAMILIES, frames=100, log=print):
    """Coordinate descent over the families; returns (gemm_config, best ms, table)."""
    sp = _spec.get_spec(spec)
    sp.pop('gemm_config', None)
    weights = _spec.make_weights(sp)
    shp = shapes(sp)
    choice = {}
    # the first engine of a process runs slower (about 0.6% on the 1B model:
    # clocks and allocations settle), so the defaults are timed twice and
    # the second run is the baseline
    present = []
    time_frames(sp, weights, frames, names=present)
    base = time_frames(sp, weights, frames)
    log(f'[tune] {sp["name"]}: engine defaults {base:.4f} ms/frame')
    best_ms, table = base, [('defaults', base)]
    for fam in families:
        if not all(n in present for n in entry_names(sp, fam)):
            # e.g. the O-projection where it runs inside the attention launch
            log(f'[tune] {fam}: no such GEMM in this plan, skipped')
            continue
        M, N, K, kind, batch = shp[fam]
        best_c = None
        for c in candidates(M, N, K, kind, batch):
            trial = dict(choice, **{fam: c})
            ms = time_frames(dict(sp, gemm_config=config_for(sp, trial)), weights, frames)
            table.append((f'{fam}={c[0]},{c[1]} ' + ' '.join(f'{f}={t},{s}' for f, (t, s) in choice.items()), ms))
            log(f'[tune]   {fam} tile {c[0]} split {c[1]}: {ms:.4f} ms/frame')
            if ms < best_ms:
                best_ms, best_c = ms, c
        if best_c is not None:
            choice[fam] = best_c
            log(f'[tune] {fam}: tile {best_c[0]} split {best_c[1]} -> {best_ms:.4f} ms/frame')
        else:
            log(f'[tune] {fam}: engine default kept')
    return config_for(sp, choice), best_ms, table


def _main(argv=None):
    ap = argparse.ArgumentParser(prog='python -m chestnut.tune')
    ap.add_argument('--spec', default='big_driving_1b')
    ap.add_argument('--families', default=','.join(FAMILIES))
    ap.add_argument('--frames', type=int, default=100)
    ap.add_argument('--out', default=None, help='write the gemm_config object as JSON')
    a = ap.parse_args(argv)
    fams = [f for f in a.families.split(',') if f]
    for f in fams:
        if f not in FAMILIES + SINGLE:
            raise SystemExit(f'unknown family {f!r}; choose from {FAMILIES + SINGLE}')
    cfg, ms, _ = tune(a.spec, fams, a.frames)
    print(f'[tune] best {ms:.4f} ms/frame ({1e3 / ms:.1f} fps)')
    if a.out:
        with open(a.out, 'w') as fh:
            json.dump(cfg, fh)
    return 0


if __name__ == '__main__':
    sys.exit(_main())
