"""Pins the oracle's model pieces (CPU): closed forms, invariants and
brute-force loops, plus determinism of the seeded spec."""
import numpy as np

from chestnut import spec as S
from oracle import model as M
from oracle import parse as PR


def test_layernorm_invariants():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((6, 128)) * 3 + 1
    y = M.layernorm(x, np.ones(128), np.zeros(128), 1e-5)
    np.testing.assert_allclose(y.mean(-1), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(-1), 1 - 1e-5 / x.var(-1), rtol=1e-9)
    g, b = rng.standard_normal(128), rng.standard_normal(128)
    np.testing.assert_allclose(M.layernorm(x, g, b, 1e-5), y * g + b, rtol=1e-12, atol=1e-12)


def test_softmax_rows():
    rng = np.random.default_rng(1)
    s = rng.standard_normal((4, 9)) * 10
    p = M.softmax_rows(s)
    np.testing.assert_allclose(p.sum(-1), 1, rtol=1e-12)
    np.testing.assert_allclose(M.softmax_rows(s + 7.0), p, rtol=1e-12)


def test_attention_bruteforce():
    rng = np.random.default_rng(2)
    T, H, hd = 6, 2, 4
    d = H * hd
    qkv = M.f16r(rng.standard_normal((T, 3 * d)))
    out = M.attention(qkv, H, hd)
    for h in range(H):
        for i in range(T):
            s = [sum(qkv[i, h * hd + c] * qkv[j, d + h * hd + c] for c in range(hd)) / np.sqrt(hd) for j in range(T)]
            e = np.exp(np.array(s) - max(s))
            p = M.f16r(e / e.sum())
            for c in range(hd):
                ref = M.f16r(sum(p[j] * qkv[j, 2 * d + h * hd + c] for j in range(T)))
                assert out[i, h * hd + c] == ref


def test_attention_uniform_keys_average_values():
    """Identical keys -> uniform attention -> mean of the values."""
    T, H, hd = 8, 1, 4
    qkv = np.zeros((T, 12), np.float32)
    qkv[:, 0:4] = 0.5
    qkv[:, 4:8] = 0.25
    qkv[:, 8:12] = np.arange(T * 4).reshape(T, 4)
    out = M.attention(qkv, H, hd)
    np.testing.assert_allclose(out, np.tile(qkv[:, 8:12].mean(0), (T, 1)), rtol=1e-3)


def _tiny_weights():
    sp = S.get_spec('tiny')
    return sp, S.make_weights(sp)


def test_stem_conv_bruteforce_one_output():
    sp, w = _tiny_weights()
    rng = np.random.default_rng(3)
    img = rng.integers(0, 256, (12, 128, 256), dtype=np.uint8)
    out = M.stem_forward(img, w, 1, 1)          # first layer only, stream 1
    Wc = w['stem.0.w'][1].astype(np.float64)    # [Co, 3, 3, Ci]
    bc = w['stem.0.b'][1].astype(np.float64)
    xn = (img.astype(np.float64) - 128) / 128
    for (ho, wo, co) in [(0, 0, 0), (0, 127, 3), (63, 0, 5), (31, 77, 7), (63, 127, 1)]:
        acc = bc[co]
        for ky in range(3):
            for kx in range(3):
                y, x = 2 * ho - 1 + ky, 2 * wo - 1 + kx
                if 0 <= y < 128 and 0 <= x < 256:
                    acc += sum(Wc[co, ky, kx, c] * xn[c, y, x] for c in range(12))
        assert out[ho, wo, co] == M.f16r(max(acc, 0.0))


def test_tokens_layout():
    a = np.arange(4 * 8 * 3, dtype=np.float32).reshape(4, 8, 3)
    b = -a
    F = M.tokens_from_stem(a, b)
    assert F.shape == (3, 64)
    assert F[2, 5] == a.reshape(32, 3)[5, 2] and F[1, 32 + 7] == b.reshape(32, 3)[7, 1]


def test_gru_closed_forms():
    """z -> 1 keeps h_prev; with gates pushed to (r=1, z=0) h = tanh(gi_n + gh_n)."""
    sp, w = _tiny_weights()
    Hh = sp['hidden']
    w = dict(w)
    w['gru.bih'] = np.zeros(3 * Hh, np.float32)
    w['gru.bhh'] = np.zeros(3 * Hh, np.float32)
    w['gru.bih'][Hh:2 * Hh] = 60.0          # z = 1
    rng = np.random.default_rng(4)
    packed = rng.standard_normal(524).astype(np.float32)
    x = rng.standard_normal((64, sp['d_model'])).astype(np.float32)
    out = M.head_forward(x, packed, w, sp)
    np.testing.assert_allclose(out[-Hh:], packed[12:], rtol=1e-6, atol=1e-6)


def test_weights_deterministic_and_seeded():
    sp = S.get_spec('tiny')
    a = S.make_param(42, 'blk.0.qkv.w', (3, 4), 'f16', 'normal', 0.02)
    b = S.make_param(42, 'blk.0.qkv.w', (3, 4), 'f16', 'normal', 0.02)
    c = S.make_param(43, 'blk.0.qkv.w', (3, 4), 'f16', 'normal', 0.02)
    np.testing.assert_array_equal(a, b)
    assert not np.array_equal(a, c)
    assert S.output_size(sp) == 2185
    sl = S.output_slices(sp)
    assert sl['plan'] == slice(0, 990) and sl['hidden_state'] == slice(1673, 2185)


def test_param_counts():
    assert 38e6 < S.param_count('driving_39m') < 40e6
    assert 1.0e9 < S.param_count('big_driving_1b') < 1.1e9


def test_tiny_oracle_frames_deterministic_and_input_sensitive():
    sp, w = _tiny_weights()
    rng = np.random.default_rng(5)
    warped = rng.integers(0, 256, (2, 6, 128, 256), dtype=np.uint8)
    packed = np.zeros(524, np.float32)
    packed[8:10] = (1.0, 0.0)
    o1 = M.OracleModel(sp, w).run_frame(warped, packed)
    o2 = M.OracleModel(sp, w).run_frame(warped, packed)
    np.testing.assert_array_equal(o1, o2)
    assert np.all(np.isfinite(o1))
    o3 = M.OracleModel(sp, w).run_frame(np.full_like(warped, 220), packed)
    assert np.abs(o3 - o1).max() > 1e-4


def test_parse_mdn_closed_form():
    raw = np.arange(8, dtype=np.float64).reshape(1, 8) / 10
    mu, std = PR.parse_mdn_single(raw, (2, 2))
    np.testing.assert_allclose(mu.reshape(-1), raw[0, :4])
    np.testing.assert_allclose(std.reshape(-1), np.exp(raw[0, 4:]))
    assert PR.safe_exp(100.0) == np.exp(11.0)
    np.testing.assert_allclose(PR.sigmoid(0.0), 0.5)
    np.testing.assert_allclose(PR.softmax(np.array([[1.0, 1.0]])), [[0.5, 0.5]])


def test_parse_mdn_mhp_selects_best_hypothesis():
    # 2 hypotheses, 1 output: hypothesis 1 has the higher weight logit
    raw = np.zeros((1, 2, 5))
    raw[0, 0, :2] = [1, 2]
    raw[0, 1, :2] = [3, 4]
    raw[0, 0, 4] = -1.0
    raw[0, 1, 4] = 2.0
    mu, std, w = PR.parse_mdn_mhp(raw.reshape(1, -1), 2, 1, (2,))
    np.testing.assert_allclose(mu.reshape(-1), [3, 4])
    assert w[0, 0, 0] > w[0, 1, 0]


def test_parse_outputs_dict_closed_forms():
    """The dict-level Parser restatement on hand-built raw heads."""
    outs = {
        'plan': np.concatenate([np.arange(495) / 100.0, np.full(495, 20.0)]).reshape(1, -1),
        'lead_prob': np.zeros((1, 3)),
        'desire_pred': np.zeros((1, 32)),
        'lead': np.zeros((1, 144)),
        'hidden_state': np.arange(4.0).reshape(1, 4),
    }
    p = PR.parse_outputs(outs)
    assert p['plan'].shape == (1, 33, 15) and p['plan_stds'].shape == (1, 33, 15)
    np.testing.assert_allclose(p['plan'].reshape(-1), np.arange(495) / 100.0)
    np.testing.assert_allclose(p['plan_stds'], np.exp(11.0))           # safe_exp clips at 11
    np.testing.assert_allclose(p['lead_prob'], 0.5)                    # sigmoid(0)
    np.testing.assert_allclose(p['desire_pred'], 1 / 8)                # uniform groups of 8
    assert p['desire_pred'].shape == (1, 4, 8)
    assert p['lead'].shape == (1, 3, 6, 4)                             # 144 values: not multi-hypothesis
    np.testing.assert_array_equal(p['hidden_state'], outs['hidden_state'])


def test_parse_outputs_lead_mhp():
    """2 hypotheses x (24 mu | 24 std | 3 weight logits): selection 0 goes to
    hypothesis 1 (logit ln 3 vs 0: weights 1/4, 3/4), selections 1 and 2 to
    hypothesis 0."""
    raw = np.zeros((2, 51))
    raw[0, :24], raw[1, :24] = 1.0, 2.0
    raw[0, 24:48], raw[1, 24:48] = 0.0, np.log(2.0)
    raw[0, 48:] = [0.0, 1.0, 1.0]
    raw[1, 48:] = [np.log(3.0), 0.0, 0.0]
    p = PR.parse_outputs({'lead': raw.reshape(1, -1)})
    np.testing.assert_allclose(p['lead_weights'][0, :, 0], [0.25, 0.75])
    np.testing.assert_allclose(p['lead'][0, 0], 2.0)
    np.testing.assert_allclose(p['lead_stds'][0, 0], 2.0)
    np.testing.assert_allclose(p['lead'][0, 1:], 1.0)
    assert p['lead'].shape == (1, 3, 6, 4) and p['lead_hypotheses'].shape == (1, 2, 6, 4)
