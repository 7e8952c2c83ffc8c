"""Oracle restatement of image2d texel addressing.

Test infrastructure only (see oracle/__init__.py).  Integer-exact: the device
gather must match bit for bit.
"""
import numpy as np


def img_texel_zero_border(img, y, x):
    """Texel (y, x) of an image param (A rows, B texels per row, C lanes),
    OpenCL CLK_ADDRESS_CLAMP semantics (border colour = zero).

    Restates the image branch of `_addrflat` (run_pinned2.py:56-84) and the
    masked LOAD (run_pinned2.py:355-374):
        fl    = y*B + x
        fc    = clamp(fl, 0, A*B)          (upper bound inclusive, as emitted)
        valid = 0 <= x < B  and  0 <= y < A
        value = valid ? texel[fc] : 0
    For every valid (y, x), fc == fl, so the value never depends on the clamp;
    the clamp only keeps the address inside the allocation (plus one texel in
    the reference, whose bound is A*B rather than A*B-1).
    img: array [A, B, C].  Returns an array [C] of img's dtype.
    Pinned by: research/probe_sampler.py's OOB case list (tests/golden).
    """
    A, B, C = img.shape
    fl = int(y) * B + int(x)
    fc = min(max(fl, 0), A * B)
    valid = (0 <= x < B) and (0 <= y < A)
    if not valid:
        return np.zeros(C, img.dtype)
    assert fc == fl
    return img.reshape(A * B, C)[fc].copy()


def img_texel_edge_clamp(img, y, x):
    """Edge-clamp variant of the fallback path (`_rule_index`,
    run_pinned2.py:658-684): y and x are clamped into range first, so
    out-of-range reads return the nearest edge texel."""
    A, B, C = img.shape
    yc = min(max(int(y), 0), A - 1)
    xc = min(max(int(x), 0), B - 1)
    return img[yc, xc].copy()


def gather(img, yx, mode='zero'):
    """Vectorised gather: yx int [n, 2] (y, x) -> [n, C] texels."""
    img = np.asarray(img)
    A, B, C = img.shape
    yx = np.asarray(yx, np.int64).reshape(-1, 2)
    y, x = yx[:, 0], yx[:, 1]
    if mode == 'edge':
        return img[np.clip(y, 0, A - 1), np.clip(x, 0, B - 1)]
    valid = (x >= 0) & (x < B) & (y >= 0) & (y < A)
    fc = np.clip(y * B + x, 0, A * B - 1)
    out = img.reshape(A * B, C)[fc]
    out[~valid] = 0
    return out
