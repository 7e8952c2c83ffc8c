"""rocprofv3 output -> per-plan-entry tables (the KTIME/KSYNC view of a frame,
run_pinned2.py:1307-1329, 1513-1557, built from a kernel trace instead of
per-launch synchronisation) and HBM traffic of one plan entry from two PMC
passes (FETCH_SIZE, WRITE_SIZE).

Runs on the CPU over files a GPU run left behind:

    python -m chestnut.profiling frames TRACE.csv STATS.csv PLAN.json CMD > summary.md
    python -m chestnut.profiling traffic FETCH.csv WRITE.csv PMCRUN.json CMD OUT.json > summary.md
    python -m chestnut.profiling configs RUN.json TRACE.csv FETCH.csv WRITE.csv MFMA.csv CMD OUT.json > summary.md
    python -m chestnut.profiling gaps RUN.json TRACE.csv CMD OUT.json [PLAIN_RUN.json] > summary.md

PLAN.json is written by ``bench.py --dump-plan``; PMCRUN.json by
``bench.py --pmc-run FAMILY[,FAMILY...]``, which runs the first plan entry of
each family alone `reps` times after a plain device-to-device copy of known
size.  The copy calibrates both
counters: its algorithmic bytes divided by what the counter reports for it
is the factor applied to the entry's counts.
"""
import csv
import json
import re
import statistics
import sys


def family(name):
    return re.sub(r'^blk\d+\.', 'blk.', name)


def _expect(kernel):
    k = kernel.split('+')[0]
    if k.startswith('gemm'):
        return 'gemm'
    if k.startswith('gemv'):
        return 'gemv'
    if 'layernorm' in k:
        return 'layernorm'
    if k.startswith('attention'):   # attention, attention_oproj: one attention_kernel
        return 'attention'
    return k


def load_trace(path):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    return [(r['Kernel_Name'], (int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3) for r in rows]


def frames_from_trace(trace, plan):
    """Cut the dispatch sequence into frames that follow the plan in order:
    a frame starts at the plan's first kernel and every later entry must match
    the next dispatch.  An entry may launch more than one kernel: a split-K
    reduce after a non-partials GEMM, and further kernels of the same family
    (e.g. the two passes of the column mean) when the next entry is of
    another family, belong to it.  Returns per-entry durations (us) per frame."""
    first = _expect(plan[0]['kernel'])
    frames = []
    i = 0
    while i < len(trace):
        if first not in trace[i][0]:
            i += 1
            continue
        j, cur, ok = i, [], True
        for k, e in enumerate(plan):
            tok = _expect(e['kernel'])
            if j >= len(trace) or tok not in trace[j][0]:
                ok = False
                break
            us = trace[j][1]
            j += 1
            if '+splitk' in e['kernel'] and 'partials' not in e['kernel'] and j < len(trace) \
                    and 'splitk_reduce' in trace[j][0]:
                us += trace[j][1]
                j += 1
            nxt = _expect(plan[k + 1]['kernel']) if k + 1 < len(plan) else None
            while nxt != tok and j < len(trace) and tok in trace[j][0]:
                us += trace[j][1]
                j += 1
            cur.append(us)
        if ok:
            frames.append(cur)
            i = j
        else:
            i += 1
    return frames


def frames_md(trace_csv, stats_csv, plan_json, cmd, top=16):
    plan = json.load(open(plan_json))
    frames = frames_from_trace(load_trace(trace_csv), plan)
    if not frames:
        raise SystemExit('no complete frame found in the trace')
    fams = {}
    for k, e in enumerate(plan):
        fams.setdefault(family(e['name']), []).append(k)
    per_frame = [sum(f) for f in frames]
    rows = []
    for fam, idx in fams.items():
        durs = [f[k] for f in frames for k in idx]
        rows.append((fam, plan[idx[0]]['kernel'], len(idx), statistics.mean(durs), min(durs),
                     statistics.mean(durs) * len(idx)))
    rows.sort(key=lambda r: -r[5])
    tot = statistics.mean(per_frame)
    out = ['Command (run from the repository root on the MI355X box):', '', '```', cmd, '```', '',
           f'{len(frames)} complete frames found in the kernel trace (dispatches matched to the plan in order); '
           f'kernel time per frame: mean {tot:.1f} us, min {min(per_frame):.1f} us.', '',
           '| plan family | kernel | launches/frame | avg us | min us | us/frame | % frame |',
           '|---|---|---:|---:|---:|---:|---:|']
    for fam, kern, n, avg, mn, pf in rows:
        out.append(f'| {fam} | {kern} | {n} | {avg:.2f} | {mn:.2f} | {pf:.1f} | {100 * pf / tot:.1f} |')
    srows = list(csv.DictReader(open(stats_csv)))
    out += ['', 'rocprofv3 --stats (every dispatch of the run, frames and per-family timing loops alike):', '',
            '| kernel | calls | avg us | min us | max us | % time |', '|---|---:|---:|---:|---:|---:|']
    for r in srows[:top]:
        n = r['Name'].replace('(anonymous namespace)', '(anon)').replace('|', '/')
        n = n[:100] + '...' if len(n) > 100 else n
        out.append(f"| `{n}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | {float(r['MinNs']) / 1e3:.2f} | "
                   f"{float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    return '\n'.join(out) + '\n'


def load_trace_ts(path):
    """(name, start ns, end ns) of every dispatch in start order."""
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    return [(r['Kernel_Name'], int(r['Start_Timestamp']), int(r['End_Timestamp'])) for r in rows]


def _frame_spans(seg, plan):
    """Frames of the plan in a dispatch segment: (first start, last end, summed
    kernel ns) of each, found as frames_from_trace finds them."""
    trace = [(n, (e - s) / 1e3) for n, s, e in seg]
    first = _expect(plan[0]['kernel'])
    spans, i = [], 0
    while i < len(seg):
        if first not in seg[i][0]:
            i += 1
            continue
        j, ok = i, True
        for k, e in enumerate(plan):
            tok = _expect(e['kernel'])
            if j >= len(seg) or tok not in seg[j][0]:
                ok = False
                break
            j += 1
            if '+splitk' in e['kernel'] and 'partials' not in e['kernel'] and j < len(seg) \
                    and 'splitk_reduce' in seg[j][0]:
                j += 1
            nxt = _expect(plan[k + 1]['kernel']) if k + 1 < len(plan) else None
            while nxt != tok and j < len(seg) and tok in seg[j][0]:
                j += 1
        if ok:
            spans.append((seg[i][1], seg[j - 1][2], sum(seg[x][2] - seg[x][1] for x in range(i, j)), j - i))
            i = j
        else:
            i += 1
    del trace
    return spans


def gaps(run_json, trace_csv):
    """Split a kernel trace of `python -m chestnut.configs --config frames39`
    at its two marker kernels (the only ones not from this library) into the
    graph run and the plain-launch run, and per run report the frame period,
    the span of a frame's kernels, their summed time, the idle time inside a
    frame and the idle time between frames."""
    run = json.load(open(run_json))
    plan = run['plan']
    tr = load_trace_ts(trace_csv)
    marks = [i for i, r in enumerate(tr) if not _is_ck(r[0])]
    groups = []   # index after each contiguous run of marker kernels
    for i in marks:
        if groups and i == groups[-1]:
            groups[-1] = i + 1
        else:
            groups.append(i + 1)
    starts = groups[-2:]
    res = {'frames_per_mode': run['frames_per_mode']}
    for mode, a, b in ((run['modes'][0], starts[0], None), (run['modes'][1], starts[1], None)):
        end = len(tr) if mode == run['modes'][1] else next(i for i in marks if i >= a)
        sp = _frame_spans(tr[a:end], plan)
        if len(sp) < 3:
            raise SystemExit(f'{mode}: fewer than 3 frames found')
        per = [(sp[k + 1][0] - sp[k][0]) / 1e3 for k in range(len(sp) - 1)]
        span = [(e - s) / 1e3 for s, e, _, _ in sp]
        busy = [k / 1e3 for _, _, k, _ in sp]
        bound = [(sp[k + 1][0] - sp[k][1]) / 1e3 for k in range(len(sp) - 1)]
        res[mode] = {'frames': len(sp), 'dispatches_per_frame': sp[0][3], 'fps_wall': run.get(f'{mode}_fps'),
                     'period_us': statistics.mean(per), 'span_us': statistics.mean(span),
                     'kernel_us': statistics.mean(busy), 'idle_inside_us': statistics.mean(span) - statistics.mean(busy),
                     'idle_between_us': statistics.mean(bound), 'idle_between_min_us': min(bound),
                     'idle_between_max_us': max(bound)}
    return res


def gaps_md(res, cmd, plain=None):
    out = ['Commands (run from the repository root on the MI355X box):', '', '```', cmd, '```', '']
    if plain:
        out += ['Untraced run: ' + '; '.join(
            f"{m}: {plain[m + '_fps']} frames/s, host {plain.get(m + '_host_call_us')} us per frame_launch call, "
            f"launch loop {plain.get(m + '_host_loop_us_per_frame')} us per frame" for m in plain['modes']) +
            ' (the launch loop runs ahead of the GPU in both modes: the GPU bounds the frame rate).', '']
    out += [
           f"The 39M frame (BASELINE config 4) launched {res['frames_per_mode']} times back to back as one graph "
           'launch per frame, then as plain launches (ck_set_graph(0)), inputs resident; frames found in the kernel '
           'trace by matching the plan.  Period: start of a frame\'s first kernel to the next frame\'s; span: its '
           'first kernel\'s start to its last kernel\'s end; kernel: the summed dispatch durations; idle inside: span '
           'less kernel; idle between: last end of one frame to first start of the next.', '',
           '| run | frames | dispatches/frame | fps (wall, this traced run) | period us | span us | kernel us | '
           'idle inside us | idle between us (min / max) |', '|---|---:|---:|---:|---:|---:|---:|---:|---|']
    for mode in ('graph', 'eager'):
        r = res[mode]
        out.append(f"| {mode} | {r['frames']} | {r['dispatches_per_frame']} | {r['fps_wall']} | {r['period_us']:.2f} | "
                   f"{r['span_us']:.2f} | {r['kernel_us']:.2f} | {r['idle_inside_us']:.2f} | "
                   f"{r['idle_between_us']:.2f} ({r['idle_between_min_us']:.2f} / {r['idle_between_max_us']:.2f}) |")
    return '\n'.join(out) + '\n'


def _counter(path, counter):
    """[(dispatch_id, kernel_name, value)] of one counter, in dispatch order."""
    rows = [r for r in csv.DictReader(open(path)) if r['Counter_Name'].startswith(counter)]
    rows.sort(key=lambda r: int(r['Dispatch_Id']))
    return [(int(r['Dispatch_Id']), r['Kernel_Name'], float(r['Counter_Value'])) for r in rows]


def _copy_and_entries(rows, n_entries, reps):
    """The calibration copy's count and, per entry, the median count of its
    `reps` launches (the run's last n_entries * reps chestnut dispatches)."""
    copy = max(v for _, n, v in rows if 'copyBuffer' in n)
    ck = [(n, v) for _, n, v in rows if 'ck::' in n or '_ZN2ck' in n][-n_entries * reps:]
    out = []
    for k in range(n_entries):
        grp = ck[k * reps:(k + 1) * reps]
        out.append((grp[0][0], statistics.median(v for _, v in grp)))
    return copy, out


def traffic(fetch_csv, write_csv, run_json):
    run = json.load(open(run_json))
    reps, nbytes, ents = run['reps'], run['copy_bytes'], run['entries']
    cf, fe = _copy_and_entries(_counter(fetch_csv, 'FETCH_SIZE'), len(ents), reps)
    cw, we = _copy_and_entries(_counter(write_csv, 'WRITE_SIZE'), len(ents), reps)
    f_fetch = nbytes / (cf * 1024.0)
    f_write = nbytes / (cw * 1024.0)
    res = {'reps': reps, 'copy_bytes': nbytes, 'copy_fetch_kib': cf, 'copy_write_kib': cw,
           'fetch_factor': round(f_fetch, 4), 'write_factor': round(f_write, 4), 'entries': []}
    for e, (kname, ef), (_, ew) in zip(ents, fe, we):
        rb, wb = ef * 1024.0 * f_fetch, ew * 1024.0 * f_write
        res['entries'].append({'entry': e['entry'], 'family': family(e['entry']), 'kernel': kname,
                               'fetch_kib': ef, 'write_kib': ew, 'read_bytes': round(rb), 'write_bytes': round(wb),
                               'traffic_bytes': round(rb + wb), 'algorithmic_bytes': e['algorithmic_bytes']})
    return res


def traffic_md(t, cmd):
    out = ['Commands (run from the repository root on the MI355X box, one counter per pass):', '', '```', cmd, '```',
           '', f"Each plan entry runs alone {t['reps']} times after one frame (median per launch).  The counters "
           'are calibrated on a plain device-to-device copy of known size: factor = copy bytes / (counter x 1024).',
           '', '| | FETCH_SIZE (KiB) | WRITE_SIZE (KiB) | read B | written B | traffic B | algorithmic B |',
           '|---|---:|---:|---:|---:|---:|---:|',
           f"| copy of {t['copy_bytes']} B (factors {t['fetch_factor']}, {t['write_factor']}) | "
           f"{t['copy_fetch_kib']:.1f} | {t['copy_write_kib']:.1f} | | | | |"]
    for e in t['entries']:
        out.append(f"| `{e['entry']}` | {e['fetch_kib']:.1f} | {e['write_kib']:.1f} | {e['read_bytes']} | "
                   f"{e['write_bytes']} | {e['traffic_bytes']} | {round(e['algorithmic_bytes'])} |")
    return '\n'.join(out) + '\n'


PEAK_TFLOPS, PEAK_GBS, N_CU, N_SIMD, N_XCD = 2500.0, 8000.0, 256, 1024, 8
MFMA_COUNTERS = ('SQ_INSTS_VALU_MFMA_MOPS_F16', 'SQ_VALU_MFMA_BUSY_CYCLES', 'SQ_BUSY_CU_CYCLES', 'GRBM_GUI_ACTIVE')


def _is_ck(name):
    return 'ck::' in name or '_ZN2ck' in name


def _units(values, run):
    """The ck dispatches of the timed units, grouped by sequence position:
    {entry: [value per timed unit]} from a dispatch-ordered list."""
    seq, n = run['sequence'], run['units_timed']
    vals = values[-n * len(seq):]
    if len(vals) < n * len(seq):
        raise SystemExit(f'expected {n * len(seq)} dispatches, found {len(vals)}')
    skip = run.get('blocks_per_rep', 0)
    out = {e: [] for e in seq}
    for u in range(n):
        if skip and u % skip == 0:
            continue          # the first block of a pass: its ln1 has no partials to add
        for k, e in enumerate(seq):
            out[e].append(vals[u * len(seq) + k])
    return out


def _counter_all(path):
    """{counter: [(dispatch, kernel, value)]} of a counter-collection CSV."""
    out = {}
    for r in csv.DictReader(open(path)):
        out.setdefault(r['Counter_Name'], []).append((int(r['Dispatch_Id']), r['Kernel_Name'],
                                                     float(r['Counter_Value'])))
    for v in out.values():
        v.sort()
    return out


def configs(run_json, trace_csv, fetch_csv=None, write_csv=None, mfma_csv=None, extra_csvs=()):
    """Per-kernel summary of a `chestnut.configs` run: trace durations, HBM
    traffic (FETCH_SIZE / WRITE_SIZE scaled by the calibration copy), MFMA
    counters, against the algorithmic work."""
    run = json.load(open(run_json))
    rows = list(csv.DictReader(open(trace_csv)))
    rows.sort(key=lambda r: int(r['Start_Timestamp']))
    ck = [(r['Kernel_Name'], (int(r['End_Timestamp']) - int(r['Start_Timestamp'])) / 1e3) for r in rows
          if _is_ck(r['Kernel_Name'])]
    durs = _units([d for _, d in ck], run)
    names = _units([n for n, _ in ck], run)
    res = {'run': run, 'entries': {}}
    for e in run['sequence']:
        d = durs[e]
        res['entries'][e] = {'kernel': names[e][0], 'n': len(d), 'mean_us': statistics.mean(d),
                             'median_us': statistics.median(d), 'min_us': min(d)}
    passes = [(fetch_csv, ('FETCH_SIZE',)), (write_csv, ('WRITE_SIZE',)), (mfma_csv, MFMA_COUNTERS)]
    res['extra'] = []
    for path in extra_csvs:
        names_in = sorted(_counter_all(path))
        passes.append((path, tuple(names_in)))
        res['extra'] += names_in
    for path, counters in passes:
        if not path:
            continue
        allc = _counter_all(path)
        for c in counters:
            key = next((k for k in allc if k.startswith(c)), None)
            if key is None:
                continue
            seqv = allc[key]
            ckv = [v for _, n, v in seqv if _is_ck(n)]
            per = _units(ckv, run)
            for e in run['sequence']:
                res['entries'][e][c] = statistics.median(per[e])
            if c in ('FETCH_SIZE', 'WRITE_SIZE'):
                copy = max(v for _, n, v in seqv if 'copyBuffer' in n)
                res[c + '_factor'] = run['copy_bytes'] / (copy * 1024.0)
                res[c + '_copy_kib'] = copy
    return res


def configs_md(res, cmd):
    run = res['run']
    alg = run['algorithmic']
    unit_us = sum(e['median_us'] for e in res['entries'].values())
    t_min = max(run['flops'] / (PEAK_TFLOPS * 1e6), run['bytes'] / (PEAK_GBS * 1e3))
    out = [f"# BASELINE config {run['config']}: {run['workload']}", '',
           'Commands (run from the repository root on the MI355X box; the counter passes each a run of their own):',
           '', '```', cmd, '```', '',
           f"Timed: {run['units_timed']} {run['unit']}s over rotating operand copies (more than the 256 MB Infinity "
           f"Cache), after one untimed pass" + (f" and {run['warmup_ms']:.0f} ms of untimed repetitions (the "
           "GPU's clocks ramp up over the first tens of milliseconds of sustained load)"
           if run.get('warmup_ms') else '') + f".  Kernel trace: {unit_us:.2f} us per {run['unit']} (the sum of the "
           f"per-kernel medians).  Algorithmic work per {run['unit']}: {run['flops'] / 1e9:.3f} GFLOP, "
           f"{run['bytes'] / 1e6:.2f} MB; roofline floor t_min = max(flops / 2.5 PFLOP/s, bytes / 8 TB/s) = "
           f"{t_min:.2f} us, so the {run['unit']} runs at {t_min / unit_us:.3f} of its roofline.  (The HIP-event "
           f"time of the traced run, {run['us_per_unit']:.2f} us per {run['unit']}, includes the tracer's own "
           'per-launch host cost.)', '']
    if 'split_k' in run:
        out += [f"Planner choice: tile {run['tile']}, split-K {run['split_k']}, workspace {run['workspace_bytes']} B.",
                '']
    out += ['| kernel | dispatches | median us | mean us | min us | algorithmic | achieved | fraction of peak |',
            '|---|---:|---:|---:|---:|---|---|---:|']
    for e, r in res['entries'].items():
        a = alg.get(e)
        if a and a['flops'] and a['flops'] / max(a['bytes'], 1) > PEAK_TFLOPS * 1e12 / (PEAK_GBS * 1e9):
            ach = a['flops'] / (r['median_us'] * 1e-6) / 1e12
            cols = f"{a['flops'] / 1e9:.3f} GFLOP | {ach:.1f} TFLOP/s | {ach / PEAK_TFLOPS:.3f}"
        elif a:
            ach = a['bytes'] / (r['median_us'] * 1e-6) / 1e9
            cols = f"{a['bytes'] / 1e6:.2f} MB | {ach:.0f} GB/s | {ach / PEAK_GBS:.3f}"
        else:
            cols = '(part of the GEMM) | | '
        name = r['kernel'].replace('(anonymous namespace)', '(anon)')
        name = name[:70] + '...' if len(name) > 70 else name
        out.append(f"| {e}: `{name}` | {r['n']} | {r['median_us']:.2f} | {r['mean_us']:.2f} | {r['min_us']:.2f} | "
                   f"{cols} |")
    if 'FETCH_SIZE_factor' in res and 'WRITE_SIZE_factor' in res:
        ff, wf = res['FETCH_SIZE_factor'], res['WRITE_SIZE_factor']
        out += ['', f"HBM traffic per dispatch (median), FETCH_SIZE x {ff:.4f} and WRITE_SIZE x {wf:.4f}: the "
                f"factors make the counters of a {run['copy_bytes']} B device-to-device copy read "
                f"{run['copy_bytes']} B and write {run['copy_bytes']} B (copy: {res['FETCH_SIZE_copy_kib']:.0f} / "
                f"{res['WRITE_SIZE_copy_kib']:.0f} KiB).", '',
                '| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | read B | written B | traffic B | algorithmic B | '
                'traffic / algorithmic |', '|---|---:|---:|---:|---:|---:|---:|---:|']
        for e, r in res['entries'].items():
            if 'FETCH_SIZE' not in r or 'WRITE_SIZE' not in r:
                continue
            rb, wb = r['FETCH_SIZE'] * 1024 * ff, r['WRITE_SIZE'] * 1024 * wf
            a = alg.get(e)
            ab = a['bytes'] if a else 0
            ratio = f'{(rb + wb) / ab:.2f}' if ab else ''
            out.append(f"| {e} | {r['FETCH_SIZE']:.1f} | {r['WRITE_SIZE']:.1f} | {rb:.0f} | {wb:.0f} | {rb + wb:.0f} | "
                       f"{ab:.0f} | {ratio} |")
    if any('SQ_VALU_MFMA_BUSY_CYCLES' in r for r in res['entries'].values()):
        out += ['', 'MFMA counters per dispatch (median).  MOPS_F16 x 512 is the f16 matrix work the kernel issued '
                '(it equals the algorithmic flops).  SQ_VALU_MFMA_BUSY_CYCLES sums busy cycles over the '
                f'{N_SIMD} SIMDs (1024 flop per busy cycle: one 32x32x16 MFMA, 32768 flop, holds its SIMD 32 '
                f'cycles); GRBM_GUI_ACTIVE sums the {N_XCD} XCDs (a calibration copy reads about 19.7-20.6 thousand '
                f'per us, 8 x about 2.5 GHz).  MFMA busy = MFMA_BUSY / (GUI_ACTIVE / {N_XCD} x {N_SIMD}), the share '
                'of SIMD-cycles with the matrix core busy over the dispatch as the counters see it (that window '
                f'includes the dispatch ramp); CU busy = SQ_BUSY_CU_CYCLES / (GUI_ACTIVE / {N_XCD} x {N_CU}), the '
                'share of CU-cycles with a wave resident.', '',
                '| kernel | MOPS_F16 x 512 | algorithmic flops | MFMA_BUSY_CYCLES | BUSY_CU_CYCLES | GUI_ACTIVE | '
                'MFMA busy | CU busy |', '|---|---:|---:|---:|---:|---:|---:|---:|']
        for e, r in res['entries'].items():
            if 'SQ_VALU_MFMA_BUSY_CYCLES' not in r:
                continue
            mops = r.get('SQ_INSTS_VALU_MFMA_MOPS_F16', 0) * 512
            gui = r.get('GRBM_GUI_ACTIVE', 0)
            busy = r['SQ_VALU_MFMA_BUSY_CYCLES'] / (gui / N_XCD * N_SIMD) if gui else 0
            cub = r.get('SQ_BUSY_CU_CYCLES', 0) / (gui / N_XCD * N_CU) if gui else 0
            a = alg.get(e)
            out.append(f"| {e} | {mops:.4g} | {(a['flops'] if a else 0):.4g} | {r['SQ_VALU_MFMA_BUSY_CYCLES']:.4g} | "
                       f"{r.get('SQ_BUSY_CU_CYCLES', 0):.4g} | {gui:.4g} | {busy:.3f} | {cub:.3f} |")
    if res.get('extra'):
        cols = res['extra']
        out += ['', 'Further counters per dispatch (median; `_sum` counters add all instances of the block).', '',
                '| kernel | ' + ' | '.join(cols) + ' |', '|---|' + '---:|' * len(cols)]
        for e, r in res['entries'].items():
            out.append(f'| {e} | ' + ' | '.join(f'{r.get(c, 0):.4g}' for c in cols) + ' |')
    return '\n'.join(out) + '\n'


def main(argv):
    if argv[0] == 'frames':
        sys.stdout.write(frames_md(argv[1], argv[2], argv[3], argv[4]))
    elif argv[0] == 'traffic':
        t = traffic(argv[1], argv[2], argv[3])
        with open(argv[5], 'w') as fh:
            json.dump(t, fh, indent=1)
        sys.stdout.write(traffic_md(t, argv[4]))
    elif argv[0] == 'gaps':
        res = gaps(argv[1], argv[2])
        with open(argv[4], 'w') as fh:
            json.dump(res, fh, indent=1)
        plain = json.load(open(argv[5])) if len(argv) > 5 else None
        sys.stdout.write(gaps_md(res, argv[3], plain))
    elif argv[0] == 'configs':
        # configs RUN.json TRACE.csv FETCH.csv WRITE.csv MFMA.csv CMD OUT.json [EXTRA.csv ...]
        # ('-' for a missing pass)
        opt = [None if x == '-' else x for x in argv[3:6]]
        res = configs(argv[1], argv[2], *opt, extra_csvs=argv[8:])
        with open(argv[7], 'w') as fh:
            json.dump(res, fh, indent=1)
        sys.stdout.write(configs_md(res, argv[6]))
    else:
        raise SystemExit(__doc__)


if __name__ == '__main__':
    main(sys.argv[1:])
