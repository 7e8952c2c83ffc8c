"""Closed-form pins of the oracle's synthetic-model composition (CPU).

The reference network lives only inside comma's pickle (README.md:59), so
`oracle.model.block_forward`, `embed` and `head_forward` *define* the
network the engine runs ("pre-LayerNorm" block; the
context inputs in run_policy's order, compile_modeld.py:198-221).  Every
test below chooses weights that collapse one of those functions to a value
computed here independently (uniform attention, one-hot selections, gates
saturated at 0 or 1, LayerNorm gains of zero), such that a plausible
misreading fails at least one of them:

  * post-LN instead of pre-LN, a dropped residual or bias, V taken from the
    Q or K columns, MLP order (up -> GELU -> down) changed;
  * Q and K swapped, the 1/sqrt(head_dim) scale missing, heads mixed;
  * the GRU gate order (r | z | n) changed, r applied to gi_n + gh_n, the
    final LN missing, a sum or max pool instead of the token mean;
  * the context vector's order [temporal | desire | traffic | action_t],
    the temporal GELU, or the position / bias / context terms of X0.
"""
import numpy as np

from chestnut import spec as S
from oracle import model as M
from oracle.kernels import gelu

rng0 = np.random.default_rng


_BASE = {}


def _tiny():
    """The tiny spec and a private copy of its seeded weights."""
    sp = S.get_spec('tiny')
    if not _BASE:
        _BASE.update(S.make_weights(sp))
    return sp, {k: v.copy() for k, v in _BASE.items()}


def _zero(w, *names):
    for n in names:
        w[n] = np.zeros_like(w[n])


def _mv(W, v):
    """f64 matrix-vector product of an f16/f32 weight with a vector."""
    return np.asarray(W, np.float64) @ np.asarray(v, np.float64)


# ---------------------------------------------------------------------------
# block_forward
# ---------------------------------------------------------------------------
def test_block_identity_without_output_projections():
    """O-proj and MLP-down weights and biases zero: both residual branches add
    exactly zero, so the block returns x bit for bit."""
    sp, w = _tiny()
    _zero(w, 'blk.0.o.w', 'blk.0.o.b', 'blk.0.down.w', 'blk.0.down.b')
    x = rng0(1).standard_normal((64, sp['d_model'])).astype(np.float32)
    np.testing.assert_array_equal(M.block_forward(x, w, 0, sp), x)


def test_block_uniform_attention_returns_v_bias():
    """qkv.w = 0: every token's q, k, v equal the f16 bias chunks, the scores
    are equal, softmax is uniform (1/64 is exact in f16) and attention returns
    the V bias in every row.  With MLP-down zero the block is
    x + W_o f16(b_v) + b_o, computed here from the V chunk (columns 2d..3d)."""
    sp, w = _tiny()
    d = sp['d_model']
    _zero(w, 'blk.0.qkv.w', 'blk.0.down.w', 'blk.0.down.b')
    w['blk.0.qkv.b'] = rng0(2).standard_normal(3 * d).astype(np.float32)
    x = rng0(3).standard_normal((64, d)).astype(np.float32)
    vb = M.f16r(w['blk.0.qkv.b'][2 * d:3 * d])
    delta = _mv(w['blk.0.o.w'], vb) + np.asarray(w['blk.0.o.b'], np.float64)
    want = (x.astype(np.float64) + delta).astype(np.float32)
    np.testing.assert_array_equal(M.block_forward(x, w, 0, sp), want)
    # the Q or K chunk in place of V gives something else
    for lo in (0, d):
        wrong = _mv(w['blk.0.o.w'], M.f16r(w['blk.0.qkv.b'][lo:lo + d])) + w['blk.0.o.b']
        assert np.abs(wrong - delta).max() > 1e-3


def test_block_is_pre_layernorm():
    """Both LayerNorm gains zero: pre-LN sub-layers then see the constant
    f16(beta) whatever x is, so block(x) - x is one fixed vector c for every
    row and every input, c = W_o v + b_o + W_down f16(gelu(W_up f16(beta2) +
    b_up)) + b_down, with v the V chunk of f16(W_qkv f16(beta1) + b_qkv)
    (uniform attention over identical tokens).  A post-LN block, a dropped
    residual, bias or GELU breaks the identity."""
    sp, w = _tiny()
    d = sp['d_model']
    w['blk.0.ln1.g'] = np.zeros(d, np.float32)
    w['blk.0.ln2.g'] = np.zeros(d, np.float32)
    b1, b2 = w['blk.0.ln1.b'], w['blk.0.ln2.b']
    qkv = M.f16r(_mv(w['blk.0.qkv.w'], M.f16r(b1)) + w['blk.0.qkv.b'])
    v = qkv[2 * d:3 * d].astype(np.float64)
    c1 = _mv(w['blk.0.o.w'], v) + np.asarray(w['blk.0.o.b'], np.float64)
    u = M.f16r(gelu(_mv(w['blk.0.up.w'], M.f16r(b2)) + np.asarray(w['blk.0.up.b'], np.float64)))
    c2 = _mv(w['blk.0.down.w'], u) + np.asarray(w['blk.0.down.b'], np.float64)
    for seed in (4, 5):
        x = (rng0(seed).standard_normal((64, d)) * (1 + seed)).astype(np.float32)
        got = M.block_forward(x, w, 0, sp)
        x1 = (x.astype(np.float64) + c1).astype(np.float32)
        want = (x1.astype(np.float64) + c2).astype(np.float32)
        np.testing.assert_array_equal(got, want)


def _attn_case(T=64, H=2, hd=64):
    """Head 0: every query q = (a, 0, ...); keys 0 and 1 carry s0, s1 on
    dim 0 with a*(s1-s0)/sqrt(hd) = ln 3, every other key a score 40 below,
    so P = (1/4, 3/4, 0, ...) exactly in f16.  Head 1: the same with the two
    keys' roles exchanged."""
    d = H * hd
    qkv = np.zeros((T, 3 * d), np.float32)
    a = 4.0
    s0 = 0.0
    s1 = np.log(3.0) * np.sqrt(hd) / a
    for h in range(H):
        qkv[:, h * hd] = a
        ks = np.full(T, -40.0 * np.sqrt(hd) / a)
        ks[0], ks[1] = (s0, s1) if h == 0 else (s1, s0)
        qkv[:, d + h * hd] = ks
    qkv = M.f16r(qkv)
    v = rng0(6).standard_normal((T, d))
    qkv[:, 2 * d:] = M.f16r(v)
    return qkv, d, hd


def test_attention_closed_form_scale_and_operand_roles():
    T, H, hd = 64, 2, 64
    qkv, d, _ = _attn_case(T, H, hd)
    out = M.attention(qkv, H, hd)
    v = qkv[:, 2 * d:].astype(np.float64)
    # the f16 rounding of s1 makes the weights 1/4, 3/4 only to ~1e-3
    k = qkv[:, d:2 * d].astype(np.float64)
    for h, (i0, i1) in enumerate(((0, 1), (1, 0))):
        z = 4.0 * (k[i1, h * hd] - k[i0, h * hd]) / np.sqrt(hd)
        p1 = M.f16r(np.exp(z) / (1 + np.exp(z)))
        p0 = M.f16r(1 / (1 + np.exp(z)))
        want = M.f16r(p0 * v[i0, h * hd:(h + 1) * hd] + p1 * v[i1, h * hd:(h + 1) * hd])
        for row in (0, 17, 63):
            np.testing.assert_array_equal(out[row, h * hd:(h + 1) * hd], want)
        np.testing.assert_allclose(p1, 0.75, atol=2e-3)
    # Q and K swapped: keys become identical rows -> uniform attention
    sw = qkv.copy()
    sw[:, :d], sw[:, d:2 * d] = qkv[:, d:2 * d], qkv[:, :d]
    assert np.abs(M.attention(sw, H, hd) - out).max() > 0.1
    # without the 1/sqrt(hd) scale the weights would be ~(0, 1)
    assert np.abs(out[0, :hd] - M.f16r(v[1, :hd])).max() > 0.05


# ---------------------------------------------------------------------------
# head_forward: final LN, token mean-pool, GRU (r | z | n), heads
# ---------------------------------------------------------------------------
def _head_setup(r_bias, z_bias, lnf_g=0.0):
    sp, w = _tiny()
    Hh, d = sp['hidden'], sp['d_model']
    w['gru.bih'] = rng0(7).standard_normal(3 * Hh).astype(np.float32) * 0.1
    w['gru.bhh'] = rng0(8).standard_normal(3 * Hh).astype(np.float32) * 0.1
    w['gru.bih'][0:Hh] = r_bias
    w['gru.bhh'][0:Hh] = 0.0
    w['gru.bih'][Hh:2 * Hh] = z_bias
    w['gru.bhh'][Hh:2 * Hh] = 0.0
    w['lnf.g'] = np.full(d, lnf_g, np.float32)
    packed = np.zeros(524, np.float32)
    packed[12:] = rng0(9).standard_normal(Hh).astype(np.float32)
    return sp, w, packed


def test_gru_r1_z0_gives_tanh_of_sum():
    """r -> 1, z -> 0: h = tanh(gi_n + gh_n) with pooled = beta (lnf.g = 0)."""
    sp, w, packed = _head_setup(60.0, -60.0)
    Hh = sp['hidden']
    x = rng0(10).standard_normal((64, sp['d_model'])).astype(np.float32)
    out = M.head_forward(x, packed, w, sp)
    pooled = np.asarray(w['lnf.b'], np.float64)
    gi_n = _mv(w['gru.wih'][2 * Hh:], pooled) + w['gru.bih'][2 * Hh:]
    gh_n = _mv(w['gru.whh'][2 * Hh:], packed[12:]) + w['gru.bhh'][2 * Hh:]
    h = np.tanh(gi_n + gh_n)
    np.testing.assert_allclose(out[-Hh:], h, rtol=1e-6, atol=1e-7)
    raw = _mv(w['head.w'], h.astype(np.float32)) + w['head.b']
    np.testing.assert_allclose(out[:-Hh], raw, rtol=1e-5, atol=1e-6)


def test_gru_r0_drops_the_hidden_term():
    """r -> 0, z -> 0: h = tanh(gi_n) (r multiplies W_hn h + b_hn only, not
    gi_n + gh_n, which would give tanh(0) = 0)."""
    sp, w, packed = _head_setup(-60.0, -60.0)
    Hh = sp['hidden']
    x = rng0(11).standard_normal((64, sp['d_model'])).astype(np.float32)
    out = M.head_forward(x, packed, w, sp)
    gi_n = _mv(w['gru.wih'][2 * Hh:], w['lnf.b']) + w['gru.bih'][2 * Hh:]
    np.testing.assert_allclose(out[-Hh:], np.tanh(gi_n), rtol=1e-6, atol=1e-7)
    assert np.abs(np.tanh(gi_n)).max() > 0.05


def test_final_layernorm_and_token_mean_pool():
    """lnf.g = 1, lnf.b = 0, rows x_t = s_t * v + c_t with v = +-1 (mean 0,
    variance 1) and |s_t| = 1000: LN(x_t) = sign(s_t) v to 1e-11.  With 48
    positive and 16 negative rows the token mean is v / 2 (a sum would give
    32 v, a max v).  With r -> 1 and z -> 0 the GRU then reads
    gi_n = W_in (v / 2) + b_in, which recovers the pool."""
    sp, w, packed = _head_setup(60.0, -60.0, lnf_g=1.0)
    w['lnf.b'] = np.zeros_like(w['lnf.b'])
    Hh, d = sp['hidden'], sp['d_model']
    v = np.where(np.arange(d) % 2 == 0, 1.0, -1.0)
    s = np.where(np.arange(64) < 48, 1000.0, -1000.0)
    c = rng0(12).standard_normal(64) * 5
    x = (s[:, None] * v[None, :] + c[:, None]).astype(np.float32)
    out = M.head_forward(x, packed, w, sp)
    pooled = v / 2
    gi_n = _mv(w['gru.wih'][2 * Hh:], pooled) + w['gru.bih'][2 * Hh:]
    gh_n = _mv(w['gru.whh'][2 * Hh:], packed[12:]) + w['gru.bhh'][2 * Hh:]
    np.testing.assert_allclose(out[-Hh:], np.tanh(gi_n + gh_n), rtol=1e-6, atol=1e-7)


def test_gru_gate_order_z_keeps_previous_state():
    """z -> 1 (second chunk) keeps h_prev whatever r is; z placed in the
    first or third chunk would not."""
    for r_bias in (60.0, -60.0):
        sp, w, packed = _head_setup(r_bias, 60.0)
        Hh = sp['hidden']
        x = rng0(13).standard_normal((64, sp['d_model'])).astype(np.float32)
        out = M.head_forward(x, packed, w, sp)
        np.testing.assert_allclose(out[-Hh:], packed[12:], rtol=1e-6, atol=1e-7)


# ---------------------------------------------------------------------------
# embed: X0 = tokens W_emb^T + b_emb + pos + ctx,
#        ctx = W_ctx [gelu(W_tmp feat + b_tmp) | desire | traffic | action_t] + b_ctx
# ---------------------------------------------------------------------------
def _inputs(sp, seed=14):
    r = rng0(seed)
    return {'img': r.integers(0, 256, (12, 128, 256), dtype=np.uint8),
            'big_img': r.integers(0, 256, (12, 128, 256), dtype=np.uint8),
            'features_buffer': r.standard_normal((sp['feat_hist'], sp['feat_len'])).astype(np.float32),
            'desire_pulse': (r.random((sp['desire_hist'], sp['desire_len'])) > 0.5).astype(np.float32),
            'traffic_convention': np.array([1.0, 0.0], np.float32),
            'action_t': r.uniform(-1, 1, 2).astype(np.float32)}


def test_embed_without_token_weights_is_bias_pos_ctx():
    sp, w = _tiny()
    _zero(w, 'emb.w')
    inp = _inputs(sp)
    tr = {}
    X = M.embed(inp, w, sp, trace=tr)
    want = (np.asarray(w['emb.b'], np.float64)[None, :] + np.asarray(w['pos'], np.float64)
            + np.asarray(tr['ctx'], np.float64)[None, :]).astype(np.float32)
    np.testing.assert_array_equal(X, want)


def test_embed_context_order_one_hot():
    """One-hot rows of ctx.w pick single entries of the context input:
    row 0 temporal[5], row 1 desire_pulse[3, 6], row 2 traffic[1], row 3
    action_t[0], row 4 action_t[1].  One-hot rows of tmp.w make temporal[i]
    = gelu(features[j_i] + b_tmp[i]).  emb.w = 0 exposes ctx in X0."""
    sp, w = _tiny()
    d, Td, L = sp['d_model'], sp['temporal_dim'], sp['feat_len']
    _zero(w, 'emb.w', 'ctx.w', 'tmp.w')
    n_ctx = w['ctx.w'].shape[1]
    dpos = Td + 3 * sp['desire_len'] + 6
    picks = {0: 5, 1: dpos, 2: Td + sp['desire_hist'] * sp['desire_len'] + 1,
             3: Td + sp['desire_hist'] * sp['desire_len'] + 2, 4: n_ctx - 1}
    for row, col in picks.items():
        w['ctx.w'][row, col] = 1.0
    fsel = {5: (7, 100)}                       # temporal[5] <- features[7, 100]
    for i, (a, b) in fsel.items():
        w['tmp.w'][i, a * L + b] = 1.0
    inp = _inputs(sp)
    X = M.embed(inp, w, sp)
    base = np.asarray(w['emb.b'], np.float64)[None, :] + np.asarray(w['pos'], np.float64)
    ctx = (X.astype(np.float64) - base)[:, :5]
    cb = np.asarray(w['ctx.b'], np.float64)[:5]
    temporal5 = gelu(np.float64(inp['features_buffer'][7, 100]) + np.float64(w['tmp.b'][5]))
    want = np.array([temporal5, inp['desire_pulse'][3, 6], inp['traffic_convention'][1],
                     inp['action_t'][0], inp['action_t'][1]]) + cb
    for t in (0, 31, 63):
        np.testing.assert_allclose(ctx[t], want, rtol=0, atol=2e-6)
    assert abs(temporal5) > 1e-3


def test_embed_token_weights_select_stem_channels():
    """One-hot emb.w rows pick token features: X0[t, 0] - (b + pos + ctx) is
    feature 3 (stream 0, spatial 3) of token t and X0[t, 1] feature 40
    (stream 1, spatial 8), i.e. stem channel t of each stream."""
    sp, w = _tiny()
    w['emb.w'] = np.zeros_like(w['emb.w'])
    w['emb.w'][0, 3] = 1.0
    w['emb.w'][1, 40] = 1.0
    inp = _inputs(sp)
    tr = {}
    X = M.embed(inp, w, sp, trace=tr)
    rest = (np.asarray(w['emb.b'], np.float64)[None, :] + np.asarray(w['pos'], np.float64)
            + np.asarray(tr['ctx'], np.float64)[None, :])
    got = X.astype(np.float64) - rest
    s0 = tr['stem0'].reshape(-1, tr['stem0'].shape[-1])     # [spatial, channel]
    s1 = tr['stem1'].reshape(-1, tr['stem1'].shape[-1])
    np.testing.assert_allclose(got[:, 0], s0[3, :], atol=2e-6)
    np.testing.assert_allclose(got[:, 1], s1[8, :], atol=2e-6)
    assert np.abs(s0[3]).max() > 0
