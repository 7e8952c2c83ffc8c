"""The model pins have teeth: plausible mistakes planted in a copy of
oracle/model.py (on the CPU, never in the product) each fail at least one of
the closed-form pin tests in test_oracle_model_pins.py."""
import importlib.util
import os
import types

import pytest

import oracle
from oracle import model as _M

import test_oracle_model_pins as PINS

SRC = open(_M.__file__).read()

# name -> (original text, planted mistake)
MUTANTS = {
    'no_pre_ln': ("    h = f16r(layernorm(x, weights[p + 'ln1.g'], weights[p + 'ln1.b'], eps)).astype(acc)",
                  "    h = f16r(x).astype(acc)"),
    'no_attn_residual': ("x = (x.astype(acc) + (a @ _w(weights, p + 'o.w', acc).T",
                         "x = (0 * x.astype(acc) + (a @ _w(weights, p + 'o.w', acc).T"),
    'no_o_bias': ("(a @ _w(weights, p + 'o.w', acc).T + np.asarray(weights[p + 'o.b'], acc))",
                  "(a @ _w(weights, p + 'o.w', acc).T)"),
    'v_from_k_columns': ("qkv[:, d:2 * d].astype(acc), qkv[:, 2 * d:3 * d].astype(acc)",
                         "qkv[:, d:2 * d].astype(acc), qkv[:, d:2 * d].astype(acc)"),
    'q_k_swapped': ("s = (q[:, sl] @ k[:, sl].T) * scale", "s = (k[:, sl] @ q[:, sl].T) * scale"),
    'no_score_scale': ("scale = 1.0 / np.sqrt(head_dim)", "scale = 1.0"),
    'no_mlp_gelu': ("u = f16r(gelu((h2 @", "u = f16r(((h2 @"),
    'r_on_gi_plus_gh': ("n = np.tanh(gi[2 * Hh:3 * Hh] + r * gh[2 * Hh:3 * Hh])",
                        "n = np.tanh(r * (gi[2 * Hh:3 * Hh] + gh[2 * Hh:3 * Hh]))"),
    'gates_z_r_n': ("r = sigmoid(gi[0:Hh] + gh[0:Hh])\n    z = sigmoid(gi[Hh:2 * Hh] + gh[Hh:2 * Hh])",
                    "z = sigmoid(gi[0:Hh] + gh[0:Hh])\n    r = sigmoid(gi[Hh:2 * Hh] + gh[Hh:2 * Hh])"),
    'sum_pool': ("pooled = xf.astype(np.float64).mean(axis=0)", "pooled = xf.astype(np.float64).sum(axis=0)"),
    'no_final_ln': ("xf = layernorm(x, weights['lnf.g'], weights['lnf.b'], eps).astype(np.float32)", "xf = x"),
    'context_order': ("np.asarray(inputs['traffic_convention'], np.float32),\n"
                      "                             np.asarray(inputs['action_t'], np.float32)",
                      "np.asarray(inputs['action_t'], np.float32),\n"
                      "                             np.asarray(inputs['traffic_convention'], np.float32)"),
    'no_temporal_gelu': ("tmp = gelu(np.asarray(weights['tmp.w']", "tmp = (np.asarray(weights['tmp.w']"),
    'no_position_term': ("+ np.asarray(weights['emb.b'], acc) + _w(weights, 'pos', acc) + ctx.astype(acc))",
                         "+ np.asarray(weights['emb.b'], acc) + ctx.astype(acc))"),
    'streams_swapped': ("F = tokens_from_stem(out0, out1)", "F = tokens_from_stem(out1, out0)"),
}


def _mutant(name):
    a, b = MUTANTS[name]
    assert SRC.count(a) == 1, f'mutant {name}: anchor text not found once in oracle/model.py'
    spec = importlib.util.spec_from_loader(f'oracle.model_{name}', loader=None)
    mod = importlib.util.module_from_spec(spec)
    mod.__package__ = 'oracle'
    mod.__file__ = os.path.join(os.path.dirname(oracle.__file__), f'model_{name}.py')
    exec(compile(SRC.replace(a, b), mod.__file__, 'exec'), mod.__dict__)
    return mod


PIN_TESTS = [getattr(PINS, n) for n in dir(PINS) if n.startswith('test_')]


def test_unmutated_oracle_passes_every_pin():
    for t in PIN_TESTS:
        t()


@pytest.mark.parametrize('name', sorted(MUTANTS))
def test_planted_mistake_is_caught(name, monkeypatch):
    monkeypatch.setattr(PINS, 'M', _mutant(name))
    failed = []
    for t in PIN_TESTS:
        try:
            t()
        except AssertionError:
            failed.append(t.__name__)
    assert failed, f'no pin test fails when oracle/model.py has the mistake {name!r}'
