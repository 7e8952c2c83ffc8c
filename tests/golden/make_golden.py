"""Writes the golden fixtures under tests/golden/.

Every vector here is built from the test vectors the reference's own probes
use (read as text, never imported or run) or by brute force written
independently of oracle/:

wmma_consumer_kat.npz  consumer_probe.py:55-66, 142-171 -- every lane stages
                       f16 bit pattern lane*8+j+1 as both its A and B element
                       j; D = A @ B under the RDNA4 fragment map; C = 0.
mma_rowcol_kat.npz     mma_probe.py:86-95 extended from 16x8x8 to 16x16x16:
                       A[r,k] = bits(r*16+k), B[k,n] = bits(n*16+k).
sampler_kat.json       research/probe_sampler.py:12-54 -- 2x1 RGBA f32 image
                       [1..8]; reads at x=-1, x=2, y=-1, y=1 (out of range)
                       and (0,0), (1,0) (in range).  Expected values are the
                       CLK_ADDRESS_CLAMP border-colour rule stated at
                       run_pinned2.py:1203-1204 and in the probe's docstring.
pack_kat.npz           hand-built YUV planes whose bytes encode (plane, row,
                       col); expected 6-channel packing by a per-pixel loop
                       (video_check.py:27-32).
i420_kat.npz           hand-built I420 frame; expected frames_to_tensor output
                       by a per-pixel loop (compile_modeld.py:83-92).
queue_kat.npz          12 frames of tiny seeded inputs through the four policy
                       queues, expected samples from a list-based simulation
                       of shift_and_sample / sample_skip / sample_desire
                       (compile_modeld.py:166-176) with tiny shapes.

Run: python tests/golden/make_golden.py   (deterministic; rewrites the files)
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def kj(t, j):
    """RDNA4 fragment map as written in consumer_probe.py:14-19."""
    if j < 4:
        return j if t < 16 else j + 4
    return j + 4 if t < 16 else j + 8


def wmma_consumer_kat():
    vbits = np.zeros((32, 8), np.uint16)
    for lane in range(32):
        for j in range(8):
            vbits[lane, j] = lane * 8 + j + 1
    vf = vbits.view(np.float16).astype(np.float64)
    A = np.zeros((16, 16))
    B = np.zeros((16, 16))
    for lane in range(32):
        for j in range(8):
            k = kj(lane, j)
            A[lane % 16, k] = vf[lane, j]
            B[k, lane % 16] = vf[lane, j]
    D = A @ B
    dfrag = np.zeros((32, 8))
    for lane in range(32):
        for e in range(8):
            dfrag[lane, e] = D[(lane // 16) * 8 + e, lane % 16]
    np.savez(os.path.join(HERE, 'wmma_consumer_kat.npz'), fragA=vbits, fragB=vbits,
             fragC=np.zeros((32, 8), np.float32), D=D, Dfrag=dfrag)


def mma_rowcol_kat():
    bits = np.arange(256, dtype=np.uint16)
    f = bits.view(np.float16)
    A = np.empty((16, 16), np.float16)
    B = np.empty((16, 16), np.float16)
    for r in range(16):
        for k in range(16):
            A[r, k] = f[r * 16 + k]
    for k in range(16):
        for n in range(16):
            B[k, n] = f[n * 16 + k]
    D = A.astype(np.float64) @ B.astype(np.float64)
    np.savez(os.path.join(HERE, 'mma_rowcol_kat.npz'), A=A.view(np.uint16), B=B.view(np.uint16), D=D)


def sampler_kat():
    data = [1, 2, 3, 4, 5, 6, 7, 8]      # 2 texels x RGBA, one row
    cases = [  # (x, y) as the probe passes int2(x, y), expected RGBA
        ((-1, 0), [0, 0, 0, 0]),
        ((2, 0), [0, 0, 0, 0]),
        ((0, -1), [0, 0, 0, 0]),
        ((0, 1), [0, 0, 0, 0]),
        ((0, 0), [1, 2, 3, 4]),
        ((1, 0), [5, 6, 7, 8]),
    ]
    with open(os.path.join(HERE, 'sampler_kat.json'), 'w') as fh:
        json.dump({'height': 1, 'width': 2, 'lanes': 4, 'data': data,
                   'cases': [{'x': c[0][0], 'y': c[0][1], 'expect': c[1]} for c in cases]}, fh, indent=1)


def pack_kat():
    H, W = 8, 12
    Y = np.zeros((H, W), np.uint8)
    U = np.zeros((H, W), np.uint8)
    V = np.zeros((H, W), np.uint8)
    for r in range(H):
        for c in range(W):
            Y[r, c] = (r * W + c) % 251
            U[r, c] = (100 + 3 * r + 7 * c) % 256
            V[r, c] = (200 + 5 * r + 11 * c) % 256
    out = np.zeros((6, H // 2, W // 2), np.uint8)
    for i in range(H // 2):
        for j in range(W // 2):
            out[0, i, j] = Y[2 * i, 2 * j]
            out[1, i, j] = Y[2 * i + 1, 2 * j]
            out[2, i, j] = Y[2 * i, 2 * j + 1]
            out[3, i, j] = Y[2 * i + 1, 2 * j + 1]
            out[4, i, j] = U[2 * i, 2 * j]
            out[5, i, j] = V[2 * i, 2 * j]
    np.savez(os.path.join(HERE, 'pack_kat.npz'), Y=Y, U=U, V=V, out=out)


def i420_kat():
    H, W = 8, 12                       # Y is H x W; U, V are (H/2) x (W/2) each
    frame = np.zeros((H * 3 // 2, W), np.uint8)
    for r in range(H * 3 // 2):
        for c in range(W):
            frame[r, c] = (r * 17 + c * 3) % 256
    out = np.zeros((6, H // 2, W // 2), np.uint8)
    u_flat = [frame[r, c] for r in range(H, H + H // 4) for c in range(W)]
    v_flat = [frame[r, c] for r in range(H + H // 4, H + H // 2) for c in range(W)]
    for i in range(H // 2):
        for j in range(W // 2):
            out[0, i, j] = frame[2 * i, 2 * j]
            out[1, i, j] = frame[2 * i + 1, 2 * j]
            out[2, i, j] = frame[2 * i, 2 * j + 1]
            out[3, i, j] = frame[2 * i + 1, 2 * j + 1]
            out[4, i, j] = u_flat[i * (W // 2) + j]
            out[5, i, j] = v_flat[i * (W // 2) + j]
    np.savez(os.path.join(HERE, 'i420_kat.npz'), frame=frame, out=out)


def queue_kat():
    """Tiny shapes: img 6x2x3 per frame, 2 frames sampled with FS=4 (5 slots);
    feat 3 entries of width 2 (12 slots); desire 3 groups of width 2 (12 slots)."""
    fs, n_img, feat_hist, feat_len, des_hist, des_len = 4, 2, 3, 2, 3, 2
    rng = np.random.default_rng(7)
    nf = 12
    img_slots = [np.zeros((6, 2, 3), np.uint8) for _ in range(fs * (n_img - 1) + 1)]
    feat_slots = [np.zeros(feat_len, np.float32) for _ in range(fs * feat_hist)]
    des_slots = [np.zeros(des_len, np.float32) for _ in range(fs * des_hist)]
    frames, packeds, exp_img, exp_feat, exp_des = [], [], [], [], []
    for _ in range(nf):
        f = rng.integers(0, 256, (6, 2, 3), dtype=np.uint8)
        pk = rng.standard_normal(des_len + 4 + feat_len).astype(np.float32)
        frames.append(f)
        packeds.append(pk)
        img_slots = img_slots[1:] + [f]
        des_slots = des_slots[1:] + [pk[0:des_len]]
        feat_slots = feat_slots[1:] + [pk[des_len + 4:]]
        exp_img.append(np.concatenate([img_slots[i] for i in range(0, len(img_slots), fs)]))
        exp_feat.append(np.stack([feat_slots[i] for i in range(0, len(feat_slots), fs)]))
        groups = []
        for g in range(des_hist):
            m = des_slots[g * fs].copy()
            for t in range(1, fs):
                m = np.maximum(m, des_slots[g * fs + t])
            groups.append(m)
        exp_des.append(np.stack(groups))
    np.savez(os.path.join(HERE, 'queue_kat.npz'), frames=np.stack(frames), packed=np.stack(packeds),
             img=np.stack(exp_img), feat=np.stack(exp_feat), desire=np.stack(exp_des),
             shape=np.array([fs, n_img, feat_hist, feat_len, des_hist, des_len]))


if __name__ == '__main__':
    wmma_consumer_kat()
    mma_rowcol_kat()
    sampler_kat()
    pack_kat()
    i420_kat()
    queue_kat()
    print('golden fixtures written to', HERE)
