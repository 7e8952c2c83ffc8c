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
