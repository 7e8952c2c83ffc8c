"""Oracle restatement of the output decode (parse_model_outputs.py).

Test infrastructure only (see oracle/__init__.py).
"""
import numpy as np


def safe_exp(x):
    """exp(min(x, 11)) (parse_model_outputs.py:4-6)."""
    return np.exp(np.minimum(np.asarray(x, np.float64), 11.0))


def sigmoid(x):
    """1 / (1 + safe_exp(-x)) (parse_model_outputs.py:8-9)."""
    return 1.0 / (1.0 + safe_exp(-np.asarray(x, np.float64)))


def softmax(x, axis=-1):
    """max-shifted softmax (parse_model_outputs.py:11-18)."""
    x = np.asarray(x, np.float64)
    x = x - x.max(axis=axis, keepdims=True)
    e = safe_exp(x)
    return e / e.sum(axis=axis, keepdims=True)


def parse_mdn_single(raw, out_shape):
    """`parse_mdn` with in_N = out_N = 0 (parse_model_outputs.py:43-84):
    raw [B, 2n] -> mu = raw[:, :n], std = safe_exp(raw[:, n:2n]), each
    reshaped to (B,) + out_shape."""
    raw = np.asarray(raw, np.float64)
    raw = raw.reshape(raw.shape[0], 1, -1)
    n = raw.shape[2] // 2
    mu = raw[:, :, :n]
    std = safe_exp(raw[:, :, n:2 * n])
    shape = (raw.shape[0],) + tuple(out_shape)
    return mu.reshape(shape), std.reshape(shape)


def parse_mdn_mhp(raw, in_N, out_N, out_shape, return_hypotheses=False):
    """`parse_mdn` with in_N > 1 hypotheses (parse_model_outputs.py:50-75).
    Returns (mu, std, weights) of the selections, plus (hypothesis mu,
    hypothesis std) in the Parser's order when return_hypotheses."""
    raw = np.asarray(raw, np.float64)
    raw = raw.reshape(raw.shape[0], in_N, -1)
    n = (raw.shape[2] - out_N) // 2
    mu = raw[:, :, :n].copy()
    std = safe_exp(raw[:, :, n:2 * n])
    w = np.zeros((raw.shape[0], in_N, out_N))
    for i in range(out_N):
        w[:, :, i - out_N] = softmax(raw[:, :, i - out_N], axis=-1)
    if out_N == 1:
        for f in range(w.shape[0]):
            idx = np.argsort(w[f][:, 0])[::-1]
            w[f] = w[f][idx]
            mu[f] = mu[f][idx]
            std[f] = std[f][idx]
    mu_f = np.zeros((raw.shape[0], out_N, n))
    std_f = np.zeros((raw.shape[0], out_N, n))
    for f in range(w.shape[0]):
        for h in range(out_N):
            idx = np.argsort(w[f, :, h])[::-1]
            mu_f[f, h] = mu[f, idx[0]]
            std_f[f, h] = std[f, idx[0]]
    shape = (raw.shape[0], out_N) + tuple(out_shape) if out_N > 1 else (raw.shape[0],) + tuple(out_shape)
    if return_hypotheses:
        hs = (raw.shape[0], in_N) + tuple(out_shape)
        return mu_f.reshape(shape), std_f.reshape(shape), w, mu.reshape(hs), std.reshape(hs)
    return mu_f.reshape(shape), std_f.reshape(shape), w


# The Parser's per-head calls (parse_model_outputs.py:95-115) with the
# ModelConstants shapes they pass (constants.py:8-57).
MDN_HEADS = {'pose': (6,), 'wide_from_device_euler': (3,), 'road_transform': (6,),
             'lane_lines': (4, 33, 2), 'road_edges': (2, 33, 2), 'plan': (33, 15)}
SIGMOID_HEADS = ('lane_lines_prob', 'meta', 'lead_prob')
SOFTMAX_HEADS = {'desire_pred': (4, 8), 'desire_state': (8,)}
LEAD_MDN_LEN = 2 * 3 * 6 * 4


def parse_outputs(outs):
    """Parser(ignore_missing=True).parse_outputs (parse_model_outputs.py:95-120)
    on {name: raw array (1, len)}; heads the Parser does not name stay raw."""
    outs = {k: np.asarray(v, np.float64) for k, v in outs.items()}
    for name, shape in MDN_HEADS.items():
        if name in outs:
            outs[name], outs[name + '_stds'] = parse_mdn_single(outs[name], shape)
    for name in SIGMOID_HEADS:
        if name in outs:
            outs[name] = sigmoid(outs[name])
    for name, shape in SOFTMAX_HEADS.items():
        if name in outs:
            outs[name] = softmax(outs[name].reshape((outs[name].shape[0],) + shape), axis=-1)
    if 'lead' in outs:
        if outs['lead'].shape[1] == LEAD_MDN_LEN:       # is_mhp (parse_model_outputs.py:88-93)
            outs['lead'], outs['lead_stds'] = parse_mdn_single(outs['lead'], (3, 6, 4))
        else:
            mu, std, w, hmu, hstd = parse_mdn_mhp(outs['lead'], 2, 3, (6, 4), return_hypotheses=True)
            outs['lead'], outs['lead_stds'], outs['lead_weights'] = mu, std, w
            outs['lead_hypotheses'], outs['lead_stds_hypotheses'] = hmu, hstd
    return outs
