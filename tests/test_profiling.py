"""Host logic of chestnut.profiling on synthetic rocprofv3 CSVs (no GPU)."""
import csv
import json

from chestnut import profiling as P

PLAN = [
    {'name': 'inputs', 'kernel': 'policy_inputs', 'flops': 0, 'bytes': 10},
    {'name': 'stem0.conv', 'kernel': 'gemm_conv_relu+splitk2', 'flops': 4, 'bytes': 20},
    {'name': 'blk0.o', 'kernel': 'gemm_partials+splitk4', 'flops': 8, 'bytes': 30},
    {'name': 'blk0.ln2', 'kernel': 'add_layernorm_f16', 'flops': 0, 'bytes': 40},
    {'name': 'blk1.o', 'kernel': 'gemm_partials+splitk4', 'flops': 8, 'bytes': 30},
    {'name': 'final.pool', 'kernel': 'colmean', 'flops': 0, 'bytes': 8},
    {'name': 'gru.ih', 'kernel': 'gemv', 'flops': 2, 'bytes': 8},
    {'name': 'gru.hh', 'kernel': 'gemv', 'flops': 2, 'bytes': 8},
    {'name': 'tick', 'kernel': 'frame_tick', 'flops': 0, 'bytes': 4},
]
FRAME = [('ck::policy_inputs_kernel(args)', 1.0), ('gemm_dma_kernel<64, 64, 5, 1, 2>', 2.0),
         ('splitk_reduce_kernel<2>', 0.5), ('gemm_dma_kernel<128, 128, 4, 2, 6>', 3.0),
         ('layernorm_row_kernel<8, true, true>', 4.0), ('gemm_dma_kernel<128, 128, 4, 2, 6>', 5.0),
         ('colmean_part_kernel', 1.5), ('colmean_final_kernel', 0.5), ('gemv_kernel<6>', 1.0),
         ('gemv_kernel<1>', 2.0), ('frame_tick_kernel', 0.25)]


def _trace_csv(path, seq):
    with open(path, 'w', newline='') as fh:
        w = csv.writer(fh)
        w.writerow(['Kernel_Name', 'Start_Timestamp', 'End_Timestamp'])
        t = 1000
        for name, us in seq:
            w.writerow([name, t, t + int(us * 1000)])
            t += int(us * 1000) + 100


def test_frames_follow_plan_order(tmp_path):
    # noise before, a family-timing loop (inputs twice) between, two real frames
    seq = [('fillBuffer', 1.0)] + FRAME + [('ck::policy_inputs_kernel(args)', 1.0)] * 2 + FRAME
    _trace_csv(tmp_path / 't.csv', seq)
    frames = P.frames_from_trace(P.load_trace(tmp_path / 't.csv'), PLAN)
    assert len(frames) == 2
    # the reduce belongs to stem0.conv, both column-mean passes to final.pool,
    # and the two GEMVs stay separate entries
    assert frames[0] == [1.0, 2.5, 3.0, 4.0, 5.0, 2.0, 1.0, 2.0, 0.25]


def test_frames_reject_mismatch(tmp_path):
    bad = FRAME[:4] + [('attention_kernel', 1.0)] + FRAME[5:]   # blk0.ln2 replaced
    _trace_csv(tmp_path / 't.csv', bad)
    assert P.frames_from_trace(P.load_trace(tmp_path / 't.csv'), PLAN) == []


def test_fused_attention_entry_matches_the_attention_kernel(tmp_path):
    # attention with the O-projection inside is one attention_kernel dispatch
    plan = [{'name': 'blk0.attn', 'kernel': 'attention_oproj', 'flops': 1, 'bytes': 1},
            {'name': 'blk0.ln2', 'kernel': 'add_layernorm_f16', 'flops': 0, 'bytes': 1}]
    seq = [('_ZN2ck12_GLOBAL__N_116attention_kernelILi64ELi4ELb1ELi1ELi4EEEvPKDF16_', 3.0),
           ('layernorm_wave_kernel<true, 8>', 2.0)]
    _trace_csv(tmp_path / 't.csv', seq)
    assert P.frames_from_trace(P.load_trace(tmp_path / 't.csv'), plan) == [[3.0, 2.0]]


def test_frames_md_families(tmp_path):
    _trace_csv(tmp_path / 't.csv', FRAME)
    with open(tmp_path / 's.csv', 'w', newline='') as fh:
        w = csv.writer(fh)
        w.writerow(['Name', 'Calls', 'AverageNs', 'MinNs', 'MaxNs', 'Percentage'])
        w.writerow(['gemm_dma_kernel', 3, 3000, 2000, 5000, 60.0])
    json.dump(PLAN, open(tmp_path / 'p.json', 'w'))
    md = P.frames_md(tmp_path / 't.csv', tmp_path / 's.csv', tmp_path / 'p.json', 'cmd')
    assert '| blk.o | gemm_partials+splitk4 | 2 | 4.00 | 3.00 | 8.0 |' in md


def _counter_csv(path, counter, seq):
    with open(path, 'w', newline='') as fh:
        w = csv.writer(fh)
        w.writerow(['Dispatch_Id', 'Kernel_Name', 'Counter_Name', 'Counter_Value'])
        for i, (name, v) in enumerate(seq):
            w.writerow([i + 1, name, counter, v])


def test_traffic_calibration(tmp_path):
    # copy of 1 MiB reads as 512 KiB fetched (factor 2) and 1024 KiB written (factor 1)
    fetch = [('ck::x', 1.0), ('__amd_rocclr_copyBuffer', 512.0)] + [('ck::gemm', 100.0)] * 3 + \
            [('ck::attn', 10.0), ('ck::attn', 12.0), ('ck::attn', 11.0)]
    write = [('ck::x', 1.0), ('__amd_rocclr_copyBuffer', 1024.0)] + [('ck::gemm', 50.0)] * 3 + \
            [('ck::attn', 4.0)] * 3
    _counter_csv(tmp_path / 'f.csv', 'FETCH_SIZE', fetch)
    _counter_csv(tmp_path / 'w.csv', 'WRITE_SIZE', write)
    run = {'reps': 3, 'copy_bytes': 1 << 20,
           'entries': [{'entry': 'blk0.down', 'algorithmic_bytes': 1.0}, {'entry': 'blk0.attn', 'algorithmic_bytes': 2.0}]}
    json.dump(run, open(tmp_path / 'r.json', 'w'))
    t = P.traffic(tmp_path / 'f.csv', tmp_path / 'w.csv', tmp_path / 'r.json')
    assert t['fetch_factor'] == 2.0 and t['write_factor'] == 1.0
    d, a = t['entries']
    assert d['family'] == 'blk.down' and d['traffic_bytes'] == 100 * 1024 * 2 + 50 * 1024
    assert a['family'] == 'blk.attn' and a['read_bytes'] == 11 * 1024 * 2


def _trace_ts_csv(path, seq):
    """seq: (name, start us, end us)."""
    with open(path, 'w', newline='') as fh:
        w = csv.writer(fh)
        w.writerow(['Kernel_Name', 'Start_Timestamp', 'End_Timestamp'])
        for name, s, e in seq:
            w.writerow([name, int(s * 1000), int(e * 1000)])


def test_gaps_split_runs_at_markers(tmp_path):
    """The frames39 trace: warm-up frames, a torch marker, graph frames, a
    marker, plain-launch frames; per run the frame period, span, kernel time
    and the idle time inside and between frames."""
    plan = [{'name': 'inputs', 'kernel': 'gemv', 'flops': 0, 'bytes': 1},
            {'name': 'decode', 'kernel': 'decode', 'flops': 0, 'bytes': 1}]
    seq, t = [], 0.0

    def frames(n, inside, between):
        nonlocal t
        for _ in range(n):
            seq.append(('void ck::(anonymous namespace)::gemv_kernel<6>(args)', t, t + 3.0))
            seq.append(('_ZN2ck12_GLOBAL__N_113decode_kernelEv', t + 3.0 + inside, t + 5.0 + inside))
            t += 5.0 + inside + between
    frames(2, 1.0, 1.0)                                   # warm-up
    seq.append(('void at::native::fill_kernel(x)', t, t + 1.0)); t += 2.0
    frames(4, 0.5, 6.0)                                   # graph
    seq.append(('void at::native::fill_kernel(x)', t, t + 1.0))
    seq.append(('void at::native::add_kernel(x)', t + 1.0, t + 2.0)); t += 3.0
    frames(4, 2.0, 1.5)                                   # plain launches
    _trace_ts_csv(tmp_path / 't.csv', seq)
    run = {'frames_per_mode': 4, 'modes': ['graph', 'eager'], 'plan': plan, 'graph_fps': 1.0, 'eager_fps': 2.0}
    with open(tmp_path / 'run.json', 'w') as fh:
        json.dump(run, fh)
    res = P.gaps(tmp_path / 'run.json', tmp_path / 't.csv')
    g, e = res['graph'], res['eager']
    assert g['frames'] == 4 and e['frames'] == 4 and g['dispatches_per_frame'] == 2
    assert abs(g['kernel_us'] - 5.0) < 1e-9 and abs(e['kernel_us'] - 5.0) < 1e-9
    assert abs(g['idle_inside_us'] - 0.5) < 1e-9 and abs(e['idle_inside_us'] - 2.0) < 1e-9
    assert abs(g['idle_between_us'] - 6.0) < 1e-9 and abs(e['idle_between_us'] - 1.5) < 1e-9
    assert abs(g['period_us'] - 11.5) < 1e-9 and abs(e['period_us'] - 8.5) < 1e-9
    md = P.gaps_md(res, 'CMD', dict(run, graph_host_call_us=3.0, eager_host_call_us=4.0))
    assert '| graph | 4 | 2 |' in md and 'host 3.0 us per frame_launch call' in md
