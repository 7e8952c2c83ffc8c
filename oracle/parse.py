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


def parse_mdn_mhp(raw, in_N, out_N, out_shape):
    """`parse_mdn` with in_N > 1 hypotheses (parse_model_outputs.py:50-75)."""
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
    return mu_f.reshape(shape), std_f.reshape(shape), w
