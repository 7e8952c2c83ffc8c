"""Probe harness host logic: the A/B statistics (bench_r62.py:57-65)."""
import numpy as np

from chestnut.probe import compare, fmt_times


def test_compare_identical_and_diff():
    base = {'u': np.array([1.0, 2.0, 0.0, -4.0], np.float32), 'c': np.array([3], np.uint32),
            'h': np.array([1.0, 0.5], np.float16)}
    r = compare(base, {k: v.copy() for k, v in base.items()})
    assert r['bit_identical'] and r['ndiff'] == 0 and r['maxabs'] == 0.0 and r['changed'] == []
    var = {k: v.copy() for k, v in base.items()}
    var['u'][1] = 2.5          # rel 0.25
    var['u'][2] = 7.0          # baseline zero: counted in ndiff, not in maxabs/maxrel
    var['h'][0] = np.float16(1.0009765625)   # one f16 ulp above 1
    r = compare(base, var)
    assert not r['bit_identical'] and r['ndiff'] == 3 and r['changed'] == ['u', 'h']
    assert r['maxabs'] == 0.5 and r['maxrel'] == 0.25
    assert r['per_tensor']['u'][0] == 2 and r['per_tensor']['h'][0] == 1
    # scratch left out of the totals but still reported
    r = compare(base, var, ignore=('u',))
    assert r['changed'] == ['h'] and r['ndiff'] == 1 and 'u' in r['per_tensor']
    assert r['maxrel'] < 1e-3


def test_compare_negative_zero_is_a_bit_difference():
    base = {'x': np.array([0.0], np.float32)}
    r = compare(base, {'x': np.array([-0.0], np.float32)})
    assert r['ndiff'] == 1 and r['maxabs'] == 0.0


def test_fmt_times_median_of_15():
    ts = list(range(15, 0, -1))
    assert fmt_times(ts) == 'med=8.0000ms min=1.0000ms'
