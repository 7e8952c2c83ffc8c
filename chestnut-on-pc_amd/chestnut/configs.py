"""BASELINE configs 1-3 as stand-alone workloads for timing and rocprofv3.

    python -m chestnut.configs --config 1|2|3|chain|frames39|stream [--reps N] [--warmup-ms MS] [--out PATH]

Each run first copies 256 MiB device to device (the calibration dispatch the
FETCH_SIZE / WRITE_SIZE summaries scale by), runs the config's kernels
untimed for --warmup-ms of GPU time (the GPU's clocks ramp up over the first
tens of milliseconds of sustained load), then launches them `reps` times over
rotating copies of the operands, so the streamed bytes exceed the 256 MB
Infinity Cache as in a real frame, and times them with HIP events on the
launching stream.  It writes a JSON description (what
each launch is, its algorithmic flops and bytes, the event timing) that
`python -m chestnut.profiling configs` joins with the kernel trace and the
counter passes.

  1  GEMM  A f16 [1024, 6144] x B f16 [6144, 1024] -> C f32 (N(0,1)/sqrt(6144)),
     the [K][N] B of the baseline, tile and split chosen by the planner
  2  GEMV  W f16 [3072, 12288] ~ N(0, 0.02), x f32 ~ U(-1, 1) -> f32 [3072]
  3  one pre-LN block of the 1B model (d 2048, 16 x 128 heads, T 512, MLP
     8192), x ~ N(0, 1): the plan entries blkL.ln1 .. blk(L+1).ln1 of a
     4-block engine, each block with its own 100 MB of weights
  chain  the cost of a dependent launch (ck_time_launch_chain): chains of
     1000 launches of a near-empty kernel on 1, 256 and 1024 workgroups,
     plain and as one graph; and frame-sized graphs (38 launches, the 39M
     frame's dispatch count) replayed 200 times, whose per-launch cost less
     the long chain's is the fixed cost of one graph launch
  stream  the block GEMM's operand stream without its arithmetic
     (ck_time_operand_stream) on the MLP-up shape (512 x 8192 x 2048, 128x128
     tiles): LDS-DMA with 4 and 8 waves and register loads, over 10 rotating
     operand copies (weights from HBM, as in a frame) and over one (warm in
     the Infinity Cache), beside the MLP-up GEMM itself (tile 5: 128x128, one
     K-group, bias + GELU epilogue) over the same 10 copies
  frames39  BASELINE config 4 frame by frame: the 39M engine's device-resident
     frame (ck_frame_launch) 200 times as one graph launch each, then (after
     one torch kernel that marks the switch in a kernel trace) 200 times as
     plain launches; `python -m chestnut.profiling gaps` splits a kernel
     trace of it into the two runs and reports where each frame's time goes
"""
import argparse
import json
import os
import sys
import time

import numpy as np

COPY_BYTES = 256 << 20


def _events(torch):
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def calibration_copy(torch):
    src = torch.ones(COPY_BYTES, dtype=torch.uint8, device='cuda')
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def warm(torch, fn, ms):
    """Run fn() (one untimed repetition) until about `ms` of GPU time has
    passed.  fn may return its own elapsed ms (work on another stream than
    torch's); otherwise it is timed with events on torch's current stream.
    At most 10,000 repetitions."""
    if ms <= 0:
        return 0
    e0, e1 = _events(torch)
    e0.record()
    r = fn()
    e1.record()
    torch.cuda.synchronize()
    one = r if isinstance(r, float) and r > 0 else e0.elapsed_time(e1)
    n = min(int(ms / max(one, 1e-3)) + 1, 10000)
    for _ in range(n):
        fn()
    torch.cuda.synchronize()
    return n + 1


def config1(torch, reps, warmup_ms=0):
    from . import kernels as K
    M, N, Kd = 1024, 1024, 6144
    copies = 12                       # 12 x 25 MB of operands > the 256 MB Infinity Cache
    g = torch.Generator(device='cuda').manual_seed(1)
    A = [(torch.randn(M, Kd, device='cuda', generator=g) / np.sqrt(Kd)).half() for _ in range(copies)]
    B = [(torch.randn(Kd, N, device='cuda', generator=g) / np.sqrt(Kd)).half() for _ in range(copies)]
    C = torch.empty(M, N, device='cuda')
    tile, split, nb = K.gemm_workspace(M, N, Kd, True)
    ws = torch.empty(max(nb // 4, 1), device='cuda')
    for a, b in zip(A, B):
        K.gemm(a, b, out=C, workspace=ws)
    torch.cuda.synchronize()
    warm(torch, lambda: [K.gemm(a, b, out=C, workspace=ws) for a, b in zip(A, B)], warmup_ms)
    e0, e1 = _events(torch)
    e0.record()
    for r in range(reps):
        K.gemm(A[r % copies], B[r % copies], out=C, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    flops = 2.0 * M * N * Kd
    byts = 2.0 * (M * Kd + Kd * N) + 4.0 * M * N
    # with this [K][N] B, split 2 on tile 2 finishes inside the GEMM launch;
    # other splits run a reduce launch after it
    seq = ['gemm'] + (['splitk_reduce'] if split > 1 and not (split == 2 and tile == 2) else [])
    return {'config': 1, 'workload': 'GEMM 1024x6144 @ 6144x1024 f16 -> f32 ([K][N] B)', 'tile': tile,
            'split_k': split, 'workspace_bytes': nb, 'copies': copies, 'unit': 'GEMM', 'sequence': seq,
            'units_timed': reps, 'us_per_unit': us, 'flops': flops, 'bytes': byts, 'bound': 'mfma',
            'algorithmic': {'gemm': {'flops': flops, 'bytes': byts}}}


def config2(torch, reps, warmup_ms=0):
    from . import kernels as K
    rows, Kd = 3072, 12288
    copies = 5                        # 5 x 75.5 MB > the 256 MB Infinity Cache
    g = torch.Generator(device='cuda').manual_seed(2)
    W = [(torch.randn(rows, Kd, device='cuda', generator=g) * 0.02).half() for _ in range(copies)]
    x = torch.rand(Kd, device='cuda', generator=g) * 2 - 1
    y = torch.empty(rows, device='cuda')
    for w in W:
        K.gemv(w, x, out=y)
    torch.cuda.synchronize()
    warm(torch, lambda: [K.gemv(w, x, out=y) for w in W], warmup_ms)
    e0, e1 = _events(torch)
    e0.record()
    for r in range(reps):
        K.gemv(W[r % copies], x, out=y)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    byts = 2.0 * rows * Kd + 4.0 * Kd + 4.0 * rows
    return {'config': 2, 'workload': 'GEMV W f16 [3072, 12288] . x f32 -> f32 [3072]', 'copies': copies,
            'unit': 'GEMV', 'sequence': ['gemv'], 'units_timed': reps, 'us_per_unit': us,
            'flops': 2.0 * rows * Kd, 'bytes': byts, 'bound': 'hbm',
            'algorithmic': {'gemv': {'flops': 2.0 * rows * Kd, 'bytes': byts}}}


def config3(torch, reps, warmup_ms=0):
    from . import spec as S
    from .engine import Engine
    layers = 4                        # 4 x 100 MB of block weights > the 256 MB Infinity Cache
    sp = dict(S.get_spec('big_driving_1b'), n_layers=layers, name='block4')
    eng = Engine(sp)
    try:
        rng = np.random.default_rng(42)
        x = rng.standard_normal((512, 2048)).astype(np.float32)
        eng.write('x', x)
        plan = eng.plan()
        names = [e['name'] for e in plan]
        lo, hi = names.index('blk0.ln1'), names.index('final.ln')
        idx = list(range(lo, hi))      # every block's ln1 .. down (its ln1 adds the previous down's partials)
        eng.time_launches(idx, 1)
        warm(torch, lambda: eng.time_launches(idx, 1), warmup_ms)
        ms = eng.time_launches(idx, reps)
        # one block = 7 plan entries; the first block's ln1 has no partials to add, so
        # the per-entry figures use block 1 (its ln1 adds block 0's MLP-down partials)
        b1 = [i for i in idx if names[i].startswith('blk1.')]
        seq = [names[i].split('.', 1)[1] for i in b1]
        alg = {names[i].split('.', 1)[1]: {'flops': plan[i]['flops'], 'bytes': plan[i]['bytes'],
                                           'kernel': plan[i]['kernel']} for i in b1}
        return {'config': 3, 'workload': 'pre-LN block d=2048, 16x128 heads, T=512, MLP 8192 (4 blocks, own weights)',
                'blocks_per_rep': layers, 'unit': 'block', 'sequence': seq, 'units_timed': reps * layers,
                'us_per_unit': ms * 1e3 / (reps * layers), 'flops': sum(v['flops'] for v in alg.values()),
                'bytes': sum(v['bytes'] for v in alg.values()), 'bound': 'mfma', 'algorithmic': alg}
    finally:
        eng.close()


def launch_chain(torch, reps=0, warmup_ms=0):
    import ctypes
    from ._lib import call
    stream = None   # the call runs on a stream of its own

    def us(n, wgs, mode, r):
        v = ctypes.c_float()
        call('ck_time_launch_chain', n, wgs, mode, r, ctypes.byref(v), stream)
        return round(v.value, 3)
    n = 1000
    res = {'config': 'chain', 'workload': 'dependent launches of a near-empty kernel', 'n_launches': n,
           'chain_us_per_launch': {}}
    for wgs in (1, 256, 1024):
        res['chain_us_per_launch'][str(wgs)] = {'plain': us(n, wgs, 0, 3), 'graph': us(n, wgs, 1, 3)}
    f = 38
    g_frame = us(f, 256, 1, 200)
    g_long = res['chain_us_per_launch']['256']['graph']
    res['frame_graph'] = {'launches_per_graph': f, 'replays': 200, 'graph_us_per_launch': g_frame,
                          'plain_us_per_launch': us(f, 256, 0, 200),
                          'fixed_us_per_graph_launch': round((g_frame - g_long) * f, 2)}
    return res


def operand_stream(torch, reps=0, warmup_ms=0):
    import ctypes
    from . import kernels as K
    from ._lib import call
    M, N, Kd = 512, 8192, 2048
    n = reps or 200
    res = {'config': 'stream', 'workload': 'MLP-up operand stream 512 x 8192 x 2048 (128x128 tiles, 64-wide K-steps)',
           'shape': [M, N, Kd], 'bytes_per_launch_into_cus': 256 * (128 + 128) * Kd * 2, 'us_per_launch': {}}
    names = {0: 'lds_dma_4_waves', 1: 'lds_dma_8_waves', 2: 'registers_4_waves'}
    for copies in (10, 1):
        for mode in (0, 1, 2):
            v = ctypes.c_float()
            call('ck_time_operand_stream', M, N, Kd, mode, copies, n, ctypes.byref(v), None)
            res['us_per_launch'][f'{names[mode]}_copies{copies}'] = round(v.value, 2)
    copies = 10
    g = torch.Generator(device='cuda').manual_seed(3)
    A = [(torch.randn(M, Kd, device='cuda', generator=g)).half() for _ in range(copies)]
    W = [(torch.randn(N, Kd, device='cuda', generator=g) * 0.02).half() for _ in range(copies)]
    b = torch.zeros(N, device='cuda')
    out = torch.empty(M, N, device='cuda', dtype=torch.float16)
    for r in range(n):
        K.gemm_epi(A[r % copies], W[r % copies], b, 3, out, tile=5, split_k=1)
    e0, e1 = _events(torch)
    e0.record()
    for r in range(n):
        K.gemm_epi(A[r % copies], W[r % copies], b, 3, out, tile=5, split_k=1)
    e1.record()
    torch.cuda.synchronize()
    res['us_per_launch']['gemm_mlp_up_tile5_copies10'] = round(e0.elapsed_time(e1) * 1e3 / n, 2)
    # the QKV shape (N = 6144): 128x128 tiles (192 workgroups) against 128x96 (256), 12 copies of 27 MB
    Nq = 6144
    res['qkv'] = {'shape': [M, Nq, Kd], 'us_per_launch': {}}
    for mode, tile, wgs in ((0, '128x128', 192), (3, '128x96', 256)):
        v = ctypes.c_float()
        call('ck_time_operand_stream', M, Nq, Kd, mode, 12, n, ctypes.byref(v), None)
        res['qkv']['us_per_launch'][f'{tile}_{wgs}_workgroups_copies12'] = round(v.value, 2)
    return res


def frames39(torch, reps=0, warmup_ms=300.0):
    from . import spec as S
    from .engine import Engine
    sp = S.get_spec('driving_39m')
    n = reps or 200
    res = {'config': 'frames39', 'workload': 'driving_39m frames: graph replay, then plain launches',
           'frames_per_mode': n, 'modes': ['graph', 'eager']}
    with Engine(sp) as eng:
        rng = np.random.default_rng(4)
        eng.write('warped', rng.integers(0, 256, (2, 6, sp['img_h'], sp['img_w']), dtype=np.uint8))
        p = np.zeros(sp['desire_len'] + 4 + sp['feat_len'], np.float32)
        p[8:10] = (1.0, 0.0)
        eng.write('packed', p)
        res['plan'] = eng.plan()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < warmup_ms / 1e3:
            for _ in range(50):
                eng.frame_launch()
            eng.synchronize()
        for mode in res['modes']:
            eng.set_graph(mode == 'graph')
            eng.synchronize()
            marker = torch.ones(16, device='cuda')
            marker += 1                      # one torch kernel between the runs
            torch.cuda.synchronize()
            calls = []
            t0 = time.perf_counter()
            for _ in range(n):
                c0 = time.perf_counter()
                eng.frame_launch()
                calls.append(time.perf_counter() - c0)
            t1 = time.perf_counter()
            eng.synchronize()
            t2 = time.perf_counter()
            res[f'{mode}_fps'] = round(n / (t2 - t0), 1)
            # host side: one frame_launch call, and the launch loop per frame
            # (a loop shorter than the frame period means the GPU bounds the rate)
            res[f'{mode}_host_call_us'] = round(float(np.median(calls)) * 1e6, 1)
            res[f'{mode}_host_loop_us_per_frame'] = round((t1 - t0) * 1e6 / n, 1)
    return res


def main(argv=None):
    ap = argparse.ArgumentParser(prog='python -m chestnut.configs')
    ap.add_argument('--config', required=True, choices=('1', '2', '3', 'chain', 'frames39', 'stream'))
    ap.add_argument('--reps', type=int, default=0, help='timed launches (default: 120 / 200 / 10)')
    ap.add_argument('--warmup-ms', type=float, default=300.0,
                    help='untimed repetitions for about this much GPU time before the timed ones')
    ap.add_argument('--out', default=None, help='write the run description as JSON')
    a = ap.parse_args(argv)
    import torch
    if not torch.cuda.is_available():
        raise SystemExit('chestnut.configs needs a GPU')
    calibration_copy(torch)
    t0 = time.perf_counter()
    if a.config == 'chain':
        res = launch_chain(torch)
    elif a.config == 'frames39':
        res = frames39(torch, a.reps, a.warmup_ms)
    elif a.config == 'stream':
        res = operand_stream(torch, a.reps)
    else:
        cfg = int(a.config)
        reps = a.reps or {1: 120, 2: 200, 3: 10}[cfg]
        res = {1: config1, 2: config2, 3: config3}[cfg](torch, reps, a.warmup_ms)
    res['warmup_ms'] = a.warmup_ms
    res['copy_bytes'] = COPY_BYTES
    res['wall_s'] = round(time.perf_counter() - t0, 3)
    print(json.dumps(res), flush=True)
    if a.out:
        os.makedirs(os.path.dirname(os.path.abspath(a.out)), exist_ok=True)
        with open(a.out, 'w') as fh:
            json.dump(res, fh)
    return 0


if __name__ == '__main__':
    sys.exit(main())
