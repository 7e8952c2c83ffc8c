"""rocprofv3 output -> per-plan-entry tables (the KTIME/KSYNC view of a frame,
run_pinned2.py:1307-1329, 1513-1557, built from a kernel trace instead of
per-launch synchronisation) and HBM traffic of one plan entry from two PMC
passes (FETCH_SIZE, WRITE_SIZE).

Runs on the CPU over files a GPU run left behind:

    python -m chestnut.profiling frames TRACE.csv STATS.csv PLAN.json CMD > summary.md
    python -m chestnut.profiling traffic FETCH.csv WRITE.csv PMCRUN.json CMD OUT.json > summary.md

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


def main(argv):
    if argv[0] == 'frames':
        sys.stdout.write(frames_md(argv[1], argv[2], argv[3], argv[4]))
    elif argv[0] == 'traffic':
        t = traffic(argv[1], argv[2], argv[3])
        with open(argv[5], 'w') as fh:
            json.dump(t, fh, indent=1)
        sys.stdout.write(traffic_md(t, argv[4]))
    else:
        raise SystemExit(__doc__)


if __name__ == '__main__':
    main(sys.argv[1:])
