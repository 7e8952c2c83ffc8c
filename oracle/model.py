"""Oracle frame forward of the synthetic driving model.

Test infrastructure only (see oracle/__init__.py).

The reference's network exists only inside comma's pickle (README.md:59;
run_pinned2.py:1346-1370), so the network here is the synthetic analogue the
build pins in its spec (configs 4 and 5 of the baseline).  What this module
restates from the reference is the frame's *structure*: the input stage
(compile_modeld.py:198-221 via oracle.pack), the image2d zero-border reads of
the conv stem (run_pinned2.py:56-84, 355-374), the f16-input / f32-accumulate
matrix products (run_pinned2.py:100-266) and the output vector with its
`hidden_state` recurrence (run_pinned2.py:1354, 1580).

Rounding points: every tensor the device path stores as f16 is rounded to
f16 here too (via `f16r`); everything else stays f32/f64.  Accumulations run
in `acc` precision (float64 for small configs, float32 BLAS for the 1B one).
"""
import numpy as np

from .kernels import gelu
from .pack import PolicyQueues


def f16r(x):
    """Round to f16 and return as float32 (the value the device stores)."""
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def layernorm(x, g, b, eps):
    """Row LayerNorm in float64: (x - mean) / sqrt(var + eps) * g + b."""
    x = np.asarray(x, np.float64)
    mu = x.mean(axis=-1, keepdims=True)
    xc = x - mu
    var = (xc * xc).mean(axis=-1, keepdims=True)
    return xc / np.sqrt(var + eps) * np.asarray(g, np.float64) + np.asarray(b, np.float64)


def softmax_rows(s):
    s = np.asarray(s, np.float64)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / e.sum(axis=-1, keepdims=True)


def sigmoid(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def _w(weights, name, acc):
    return np.asarray(weights[name]).astype(acc)


def stem_forward(img_u8, weights, stream, n_layers, acc=np.float64):
    """Conv stem for one input stream.

    img_u8: uint8 [C, H, W] (the sampled img / big_img).  Layer 1 reads the
    normalised image v = (u8 - 128) / 128 with a zero border; every layer is a
    3x3 stride-2 pad-1 conv + bias + ReLU whose output is stored f16 in
    [H, W, C] texel layout and read by the next layer with a zero border.
    Returns float32 [H5, W5, C5] (f16 values).
    """
    x = (np.asarray(img_u8, np.float32) - 128.0) / 128.0
    x = np.transpose(x, (1, 2, 0))                         # HWC
    for i in range(n_layers):
        Wc = _w(weights, f'stem.{i}.w', acc)[stream]       # [Co, 3, 3, Ci]
        bc = np.asarray(weights[f'stem.{i}.b'], np.float32)[stream].astype(acc)
        H, W, Ci = x.shape
        Ho, Wo = (H - 1) // 2 + 1, (W - 1) // 2 + 1
        xp = np.zeros((H + 2, W + 2, Ci), acc)
        xp[1:H + 1, 1:W + 1] = x
        cols = [xp[ky:ky + 2 * Ho:2, kx:kx + 2 * Wo:2, :] for ky in range(3) for kx in range(3)]
        patches = np.concatenate(cols, axis=-1).reshape(Ho * Wo, 9 * Ci)
        y = patches @ Wc.reshape(Wc.shape[0], 9 * Ci).T + bc
        x = f16r(np.maximum(y, 0)).reshape(Ho, Wo, -1)
    return x


def tokens_from_stem(out0, out1):
    """Channels-as-tokens: token c gets the 32 spatial values of channel c of
    stream 0 followed by those of stream 1 -> f32 [C5, 64] (f16 values)."""
    a = out0.reshape(-1, out0.shape[-1]).T
    b = out1.reshape(-1, out1.shape[-1]).T
    return np.concatenate([a, b], axis=1).astype(np.float32)


def attention(qkv, n_heads, head_dim, acc=np.float64):
    """Non-causal multi-head attention on a packed [T, 3d] f16 QKV tensor.

    S = (q k^T) / sqrt(head_dim) in f32-or-better, P = softmax(S) rounded to
    f16, O = f16(P v).  Returns f32 [T, d] (f16 values).
    Pinned by: a brute-force loop; identical keys average the values; a
    two-key closed form with weights 1/4, 3/4 per head that fails with Q and
    K swapped or the scale dropped (tests/test_oracle_model_pins.py).
    """
    T = qkv.shape[0]
    d = n_heads * head_dim
    q, k, v = qkv[:, 0:d].astype(acc), qkv[:, d:2 * d].astype(acc), qkv[:, 2 * d:3 * d].astype(acc)
    scale = 1.0 / np.sqrt(head_dim)
    out = np.zeros((T, d), np.float32)
    for h in range(n_heads):
        sl = slice(h * head_dim, (h + 1) * head_dim)
        s = (q[:, sl] @ k[:, sl].T) * scale
        p = f16r(softmax_rows(s)).astype(acc)
        out[:, sl] = f16r(p @ v[:, sl])
    return out


def block_forward(x, weights, l, spec, acc=np.float64):
    """One pre-LN transformer block on the f32 residual x [T, d]:
    x += O(attn(QKV(f16 LN1(x)))); x += down(f16 gelu(up(f16 LN2(x)))).

    Pinned by (tests/test_oracle_model_pins.py, with planted mistakes in
    tests/test_oracle_mutants.py): zero output projections return x bit for
    bit; qkv.w = 0 gives uniform attention returning the V bias (closed form
    through O-proj); LayerNorm gains of zero make block(x) - x one vector for
    every input, computed in closed form (pre-LN, both residuals, biases,
    GELU).
    """
    eps = spec.get('ln_eps', 1e-5)
    H, hd = spec['n_heads'], spec['head_dim']
    p = f'blk.{l}.'
    h = f16r(layernorm(x, weights[p + 'ln1.g'], weights[p + 'ln1.b'], eps)).astype(acc)
    qkv = f16r(h @ _w(weights, p + 'qkv.w', acc).T + np.asarray(weights[p + 'qkv.b'], acc))
    a = attention(qkv, H, hd, acc).astype(acc)
    x = (x.astype(acc) + (a @ _w(weights, p + 'o.w', acc).T + np.asarray(weights[p + 'o.b'], acc))).astype(np.float32)
    h2 = f16r(layernorm(x, weights[p + 'ln2.g'], weights[p + 'ln2.b'], eps)).astype(acc)
    u = f16r(gelu((h2 @ _w(weights, p + 'up.w', acc).T + np.asarray(weights[p + 'up.b'], acc)).astype(acc))).astype(acc)
    x = (x.astype(acc) + (u @ _w(weights, p + 'down.w', acc).T + np.asarray(weights[p + 'down.b'], acc))).astype(np.float32)
    return x


def embed(inputs, weights, spec, acc=np.float64, trace=None):
    """Stem + temporal context + token embedding -> residual X0 [T, d] f32:
    X0 = tokens W_emb^T + b_emb + pos + ctx,
    ctx = W_ctx [gelu(W_tmp feat + b_tmp) | desire | traffic | action_t] + b_ctx
    (the context inputs in run_policy's order, compile_modeld.py:198-221).

    Pinned by (tests/test_oracle_model_pins.py): emb.w = 0 gives
    b + pos + ctx per row; one-hot ctx.w / tmp.w rows select each part of the
    context input; one-hot emb.w rows select stem channels of each stream.
    """
    n_stem = len(spec['stem'])
    out0 = stem_forward(inputs['img'], weights, 0, n_stem, acc)
    out1 = stem_forward(inputs['big_img'], weights, 1, n_stem, acc)
    F = tokens_from_stem(out0, out1)
    feat = np.asarray(inputs['features_buffer'], np.float32).reshape(-1).astype(np.float64)
    tmp = gelu(np.asarray(weights['tmp.w'], np.float16).astype(np.float64) @ feat
               + np.asarray(weights['tmp.b'], np.float64)).astype(np.float32)
    ctx_in = np.concatenate([tmp,
                             np.asarray(inputs['desire_pulse'], np.float32).reshape(-1),
                             np.asarray(inputs['traffic_convention'], np.float32),
                             np.asarray(inputs['action_t'], np.float32)]).astype(np.float64)
    ctx = (np.asarray(weights['ctx.w'], np.float16).astype(np.float64) @ ctx_in
           + np.asarray(weights['ctx.b'], np.float64)).astype(np.float32)
    X = (F.astype(acc) @ _w(weights, 'emb.w', acc).T
         + np.asarray(weights['emb.b'], acc) + _w(weights, 'pos', acc) + ctx.astype(acc)).astype(np.float32)
    if trace is not None:
        trace.update(stem0=out0, stem1=out1, tokens=F, temporal=tmp, ctx=ctx, x0=X)
    return X


def head_forward(x, packed, weights, spec, trace=None):
    """Final LN + token mean-pool, GRU hidden update (gates r | z | n,
    n = tanh(gi_n + r * gh_n), h = (1 - z) n + z h_prev), linear heads.
    Returns the output vector f32 [sum(head sizes) + hidden].

    Pinned by (tests/test_oracle_model_pins.py): gates saturated by +-60
    biases (r = 1, z = 0: tanh(gi_n + gh_n); r = 0: tanh(gi_n); z = 1: h_prev
    for either r); rows whose LayerNorm is +-v give a token mean of v / 2.
    """
    eps = spec.get('ln_eps', 1e-5)
    Hh = spec['hidden']
    xf = layernorm(x, weights['lnf.g'], weights['lnf.b'], eps).astype(np.float32)
    pooled = xf.astype(np.float64).mean(axis=0)
    dl = spec.get('desire_len', 8)
    h_prev = np.asarray(packed, np.float32)[dl + 4:dl + 4 + Hh].astype(np.float64)
    gi = np.asarray(weights['gru.wih'], np.float16).astype(np.float64) @ pooled + np.asarray(weights['gru.bih'], np.float64)
    gh = np.asarray(weights['gru.whh'], np.float16).astype(np.float64) @ h_prev + np.asarray(weights['gru.bhh'], np.float64)
    r = sigmoid(gi[0:Hh] + gh[0:Hh])
    z = sigmoid(gi[Hh:2 * Hh] + gh[Hh:2 * Hh])
    n = np.tanh(gi[2 * Hh:3 * Hh] + r * gh[2 * Hh:3 * Hh])
    h = ((1.0 - z) * n + z * h_prev).astype(np.float32)
    raw = (np.asarray(weights['head.w'], np.float16).astype(np.float64) @ h.astype(np.float64)
           + np.asarray(weights['head.b'], np.float64)).astype(np.float32)
    if trace is not None:
        trace.update(pooled=pooled.astype(np.float32), hidden=h)
    return np.concatenate([raw, h]).astype(np.float32)


class OracleModel:
    """Frame-by-frame oracle with the reference's queue state.

    `run_frame(warped, packed)` mirrors run_pinned2.py:1462-1565: the queues
    are pushed and sampled, the network runs, and the flat output vector is
    returned; the caller feeds `out[hidden_state]` back into packed[12:].
    """

    def __init__(self, spec, weights, acc=np.float64):
        self.spec = spec
        self.weights = weights
        self.acc = acc
        self.queues = PolicyQueues(img_h=spec.get('img_h', 128), img_w=spec.get('img_w', 256),
                                   feat_hist=spec.get('feat_hist', 24), feat_len=spec.get('feat_len', 512),
                                   desire_hist=spec.get('desire_hist', 25), desire_len=spec.get('desire_len', 8),
                                   fs=spec.get('frame_skip', 4))
        self.trace = {}

    def run_frame(self, warped, packed):
        inputs = self.queues.step(warped, packed)
        self.trace = {'inputs': inputs}
        x = embed(inputs, self.weights, self.spec, self.acc, self.trace)
        for l in range(self.spec['n_layers']):
            x = block_forward(x, self.weights, l, self.spec, self.acc)
            self.trace[f'x{l + 1}'] = x
        return head_forward(x, packed, self.weights, self.spec, self.trace)
