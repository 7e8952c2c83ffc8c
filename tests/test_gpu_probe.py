"""Probe harness on the GPU: capture a plan entry's pre-state from a real
frame, replay it alone, A/B a GEMM configuration (r62_probe.py +
bench_r62.py behaviour, tiny spec)."""
import json

import numpy as np
import pytest

from chestnut import probe

pytestmark = pytest.mark.gpu


def test_capture_and_replay_is_bit_identical(gpu, tmp_path):
    d = tmp_path / 'up'
    m = probe.capture('tiny', 'blk0.up', str(d), frames=2, reps=5)
    assert m['kernel'].startswith('gemm') and len(m['baseline_ms']) == 5
    pre, post = np.load(d / 'pre.npz'), np.load(d / 'post.npz')
    changed = [k for k in post.files if not np.array_equal(pre[k].view(np.uint8), post[k].view(np.uint8))]
    assert changed == ['u']                      # the MLP-up GEMM writes only its output
    r = probe.bench(str(d), reps=5)
    print(f"[probe] up same config: {r}", flush=True)
    assert r['bit_identical'] and r['ndiff'] == 0 and r['resized'] == []


def test_gemm_variant_within_tolerance(gpu, tmp_path):
    d = tmp_path / 'up'
    probe.capture('tiny', 'blk0.up', str(d), reps=3)
    r = probe.bench(str(d), gemm=(4, 2), reps=3)     # 64x64 tiles, K split in two + reduce
    print(f"[probe] up tile 4 split 2: ndiff={r['ndiff']} maxrel={r['maxrel']:.2e}", flush=True)
    # u is f16: a reassociated f32 sum may round to a neighbouring f16 value
    # (relative step 2^-10 .. 2^-11), so allow two f16 steps
    assert r['changed'] in ([], ['u']) and r['maxrel'] <= 2.0 ** -8


def test_partials_consumer_replay(gpu, tmp_path):
    """The residual LayerNorm reads the split-K workspace of the GEMM before
    it: the snapshot must carry it for the replay to match."""
    d = tmp_path / 'ln2'
    probe.capture('tiny', 'blk1.ln2', str(d), reps=3)
    meta = json.load(open(d / 'meta.json'))
    assert 'ws' in meta['state']
    r = probe.bench(str(d), reps=3)
    assert r['bit_identical']


_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _mix(z):
    z = np.asarray(z, np.uint64) + np.uint64(0x9E3779B97F4A7C15)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def _host_hash(buf):
    """The tensor hash of csrc/hash.hip restated on the host from its formula:
    mix(n) + sum of per-16-byte-chunk terms + per-tail-byte terms, mod 2^64."""
    n = len(buf)
    n16 = n // 16
    with np.errstate(over='ignore'):
        w = np.frombuffer(buf[:16 * n16], '<u8').reshape(-1, 2)
        ci = np.arange(n16, dtype=np.uint64)
        acc = _mix(np.uint64(n)) + np.sum(_mix(w[:, 0] ^ _mix(2 * ci)) + _mix(w[:, 1] ^ _mix(2 * ci + 1)),
                                          dtype=np.uint64)
        for j in range(n % 16):
            acc = acc + _mix(np.uint64(buf[16 * n16 + j]) ^ _mix(np.uint64(16 * n16 + j) + np.uint64(1 << 62)))
    return int(acc)


def test_state_hashes_match_host_restatement(gpu):
    """ck_state_hashes equals the hash computed on the host from the read-back
    bytes for every state tensor; it is repeatable, and changing one element
    of one tensor changes that tensor's hash only."""
    from chestnut import Engine, spec as S
    sp = S.get_spec('tiny')
    with Engine(sp, weights=S.make_weights(sp)) as eng:
        eng.run_frame(eng.make_warped(90), eng.PACKED.copy())
        h = eng.state_hashes()
        assert h == eng.state_hashes()
        snap = eng.snapshot()
        assert set(h) == set(snap)
        for name, arr in snap.items():
            assert h[name] == _host_hash(arr.tobytes()), name
        x = snap['x'].copy()
        x[5] = x[5] + 1.0
        eng.write('x', x)
        h2 = eng.state_hashes()
        assert [n for n in h if h[n] != h2[n]] == ['x']
        x[5], x[6] = snap['x'][6], snap['x'][5]        # the same values, two swapped
        eng.write('x', x)
        assert eng.state_hashes()['x'] != h['x']


def test_fingerprint_diff_graph_eager_and_variant(gpu, tmp_path):
    """probe fingerprint + diff: warm frames replayed as a graph or as plain
    launches leave the same pre-state at every launch of the next eager
    frame; a variant GEMM configuration for one entry is named as the first
    divergent launch."""
    lines = []
    a = probe.fingerprint('tiny', str(tmp_path / 'g.json'), frames=1, warm=2, warm_mode='graph', log=lines.append)
    b = probe.fingerprint('tiny', str(tmp_path / 'e.json'), frames=1, warm=2, warm_mode='eager', log=lines.append)
    assert any(l.startswith('[ksync]') and 'pre=' in l for l in lines)
    assert probe.diff(a, b) is None
    base = probe.fingerprint('tiny', None, frames=1, log=lines.append)
    var = probe.fingerprint('tiny', None, frames=1, extra={'gemm_config': {'blk0.up': [4, 2]}}, log=lines.append)
    r = probe.diff(base, var, ignore=('ws',))
    print(f'[probe] diff with blk0.up at tile 4 split 2: {r}', flush=True)
    assert r is not None and r['launch'] == 'blk0.up' and 'u' in r['tensors']


def test_operand_stream_workload_runs(gpu):
    """ck_time_operand_stream (the block GEMM's loads without arithmetic) runs
    in all four modes on a small grid and reports a positive time per launch."""
    import ctypes
    from chestnut._lib import call
    for mode in (0, 1, 2, 3):
        v = ctypes.c_float()
        call('ck_time_operand_stream', 256, 576 if mode == 3 else 512, 320, mode, 2, 3, ctypes.byref(v), None)
        print(f'[stream] mode {mode}: {v.value:.2f} us per launch', flush=True)
        assert v.value > 0
