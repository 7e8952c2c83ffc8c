"""Synthetic driving-model specs and seeded weights.

The reference loads comma's pickles (run_pinned2.py:1346-1370), which are not
available here; the models this engine runs are the seeded random-init
analogues pinned below.  A spec is a flat JSON object the native engine
parses (`ck_create`); the parameter table is derived from it identically in
Python (`param_table`) and in C++ (engine.cpp), and a test checks the two
agree name by name.

Architecture (one frame):
  queues      img / big_img uint8 [12,128,256], desire [25,8], features [24,512]
  stem        per stream, len(stem) 3x3 stride-2 pad-1 convs with zero-border
              image reads, bias + ReLU, f16 [H,W,C] texel layout
  tokens      channels-as-tokens: token c = 32 spatial values of stem channel c
              of each stream (64 features) -> Linear(64 -> d) + pos + context
  context     gelu(W_tmp [temporal_dim x 12288] . features) -> with desire,
              traffic convention, action_t -> Linear(-> d), added to every token
  blocks      n_layers pre-LN blocks: MHA (n_heads x head_dim), MLP d_ff, GELU
  head        final LN, mean-pool over tokens, GRU(hidden) with h_prev =
              packed prev_feat, linear heads on the new hidden state
  outputs     [head outputs ..., hidden_state]
"""
import json
import zlib
from concurrent.futures import ThreadPoolExecutor

import numpy as np

DEFAULT_OUTPUTS = [['plan', 990], ['lead', 144], ['lead_prob', 3],
                   ['lane_lines', 528], ['lane_lines_prob', 8]]

_BASE = dict(img_h=128, img_w=256, n_frames=2, frame_skip=4,
             feat_len=512, feat_hist=24, desire_len=8, desire_hist=25,
             hidden=512, ln_eps=1e-5, seed=42, outputs=DEFAULT_OUTPUTS)

SPECS = {
    # conv stem 32->256, 4 blocks d=512, 8 heads, 256 tokens
    'driving_39m': dict(_BASE, name='driving_39m', stem=[32, 64, 128, 256, 256],
                        d_model=512, n_heads=8, head_dim=64, n_layers=4, d_ff=2048,
                        temporal_dim=1664),
    # 20 blocks d=2048, 16 heads x 128, MLP 8192, 512 tokens
    'big_driving_1b': dict(_BASE, name='big_driving_1b', stem=[32, 64, 128, 256, 512],
                           d_model=2048, n_heads=16, head_dim=128, n_layers=20, d_ff=8192,
                           temporal_dim=3072),
    # small spec for fast parity tests (same structure, tiny widths)
    'tiny': dict(_BASE, name='tiny', stem=[8, 16, 32, 64, 64],
                 d_model=128, n_heads=2, head_dim=64, n_layers=2, d_ff=512,
                 temporal_dim=256),
}


# NV12 geometry of a road-camera frame (1928x1208, rows padded to 2048 bytes,
# Y plane padded to 1216 rows), as openpilot's camerad hands it to modeld
# (compile_modeld.py:16-31).  A spec with a "camera" object accepts raw NV12
# frames (Engine.run_frame_nv12) and warps them on device.
ROAD_CAMERA = dict(width=1928, height=1208, stride=2048, y_height=1216)


def nv12_bytes(camera):
    """Bytes of one NV12 frame: the padded Y plane and the half-height
    interleaved UV rows (compile_modeld.py:97-104)."""
    return camera['stride'] * camera['y_height'] + (camera['height'] // 2) * camera['stride']


def get_spec(name_or_spec):
    if isinstance(name_or_spec, dict):
        return dict(name_or_spec)
    return dict(SPECS[name_or_spec])


def spec_json(spec):
    return json.dumps(get_spec(spec), separators=(',', ':'))


def output_slices(spec):
    """name -> slice into the flat output vector (heads then hidden_state)."""
    spec = get_spec(spec)
    out, off = {}, 0
    for name, n in spec['outputs']:
        out[name] = slice(off, off + n)
        off += n
    out['hidden_state'] = slice(off, off + spec['hidden'])
    return out


def output_size(spec):
    spec = get_spec(spec)
    return sum(n for _, n in spec['outputs']) + spec['hidden']


def param_table(spec):
    """Ordered list of (name, shape, dtype, init, scale).

    init: 'normal' -> mean 0, std scale; 'one_normal' -> 1 + scale * N(0,1).
    """
    s = get_spec(spec)
    d, F, Hh = s['d_model'], s['d_ff'], s['hidden']
    T = s['stem'][-1]
    n_spatial = (s['img_h'] >> len(s['stem'])) * (s['img_w'] >> len(s['stem']))
    tok_feat = 2 * n_spatial
    n_ctx = s['temporal_dim'] + s['desire_hist'] * s['desire_len'] + 4
    n_head = sum(n for _, n in s['outputs'])
    P = []
    ci = 6 * s['n_frames']
    for i, co in enumerate(s['stem']):
        P.append((f'stem.{i}.w', (2, co, 3, 3, ci), 'f16', 'normal', float(np.sqrt(2.0 / (9 * ci)))))
        P.append((f'stem.{i}.b', (2, co), 'f32', 'normal', 0.02))
        ci = co
    P.append(('emb.w', (d, tok_feat), 'f16', 'normal', 0.02))
    P.append(('emb.b', (d,), 'f32', 'normal', 0.02))
    P.append(('pos', (T, d), 'f16', 'normal', 0.02))
    P.append(('tmp.w', (s['temporal_dim'], s['feat_hist'] * s['feat_len']), 'f16', 'normal', 0.02))
    P.append(('tmp.b', (s['temporal_dim'],), 'f32', 'normal', 0.02))
    P.append(('ctx.w', (d, n_ctx), 'f16', 'normal', 0.02))
    P.append(('ctx.b', (d,), 'f32', 'normal', 0.02))
    for l in range(s['n_layers']):
        p = f'blk.{l}.'
        P += [(p + 'ln1.g', (d,), 'f32', 'one_normal', 0.02), (p + 'ln1.b', (d,), 'f32', 'normal', 0.02),
              (p + 'qkv.w', (3 * d, d), 'f16', 'normal', 0.02), (p + 'qkv.b', (3 * d,), 'f32', 'normal', 0.02),
              (p + 'o.w', (d, d), 'f16', 'normal', 0.02), (p + 'o.b', (d,), 'f32', 'normal', 0.02),
              (p + 'ln2.g', (d,), 'f32', 'one_normal', 0.02), (p + 'ln2.b', (d,), 'f32', 'normal', 0.02),
              (p + 'up.w', (F, d), 'f16', 'normal', 0.02), (p + 'up.b', (F,), 'f32', 'normal', 0.02),
              (p + 'down.w', (d, F), 'f16', 'normal', 0.02), (p + 'down.b', (d,), 'f32', 'normal', 0.02)]
    P += [('lnf.g', (d,), 'f32', 'one_normal', 0.02), ('lnf.b', (d,), 'f32', 'normal', 0.02),
          ('gru.wih', (3 * Hh, d), 'f16', 'normal', 0.02), ('gru.bih', (3 * Hh,), 'f32', 'normal', 0.02),
          ('gru.whh', (3 * Hh, Hh), 'f16', 'normal', 0.02), ('gru.bhh', (3 * Hh,), 'f32', 'normal', 0.02),
          ('head.w', (n_head, Hh), 'f16', 'normal', 0.02), ('head.b', (n_head,), 'f32', 'normal', 0.02)]
    return P


def param_count(spec):
    return sum(int(np.prod(shape)) for _, shape, _, _, _ in param_table(spec))


def make_param(seed, name, shape, dtype, init, scale):
    """One parameter from its own stream: default_rng([seed, crc32(name)])."""
    rng = np.random.default_rng([int(seed), zlib.crc32(name.encode())])
    z = rng.standard_normal(int(np.prod(shape)), dtype=np.float32).reshape(shape)
    v = z * np.float32(scale)
    if init == 'one_normal':
        v = v + np.float32(1.0)
    return v.astype(np.float16 if dtype == 'f16' else np.float32)


def make_weights(spec, seed=None, threads=8):
    """All parameters of `spec` as a dict name -> numpy array (f16 / f32)."""
    s = get_spec(spec)
    seed = s['seed'] if seed is None else seed
    table = param_table(s)
    with ThreadPoolExecutor(max_workers=max(1, threads)) as ex:
        arrs = list(ex.map(lambda p: make_param(seed, *p), table))
    return {p[0]: a for p, a in zip(table, arrs)}
