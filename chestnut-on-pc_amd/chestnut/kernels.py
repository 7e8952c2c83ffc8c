"""Per-kernel entry points on torch device tensors (probe / bench harness).

torch provides device memory and the current stream only; every computation
is a call into libchestnut.so.  Shape / dtype / contiguity are checked here,
and again natively before any launch.
"""
import ctypes

import torch

from ._lib import call


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _need(t, dtype, name):
    if not (t.is_cuda and t.dtype == dtype and t.is_contiguous()):
        raise ValueError(f'{name} must be a contiguous {dtype} CUDA tensor')


def gemv(W, x, bias=None, act=0, rows_per_wg=0, out=None):
    """y = act(W @ x + bias): W f16 [rows, K], x f32 [K] -> f32 [rows]."""
    _need(W, torch.float16, 'W')
    _need(x, torch.float32, 'x')
    rows, K = W.shape
    y = out if out is not None else torch.empty(rows, dtype=torch.float32, device=W.device)
    if bias is not None:
        _need(bias, torch.float32, 'bias')
    call('ck_gemv', _ptr(W), _ptr(x), _ptr(bias), _ptr(y), rows, K, K, act, rows_per_wg, _stream())
    return y


def gemm_workspace(M, N, K, b_kn, tile=0, split_k=0):
    t, s, nb = ctypes.c_int(tile), ctypes.c_int(split_k), ctypes.c_size_t()
    call('ck_gemm_workspace', M, N, K, 1 if b_kn else 0, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    return t.value, s.value, nb.value


def gemm(A, B, b_kn=True, bias=None, tile=0, split_k=0, out=None, workspace=None):
    """C f32 = A @ B: A f16 [M, K]; B f16 [K, N] (b_kn) or [N, K]."""
    _need(A, torch.float16, 'A')
    _need(B, torch.float16, 'B')
    M, K = A.shape
    N = B.shape[1] if b_kn else B.shape[0]
    tile, split_k, nb = gemm_workspace(M, N, K, b_kn, tile, split_k)
    C = out if out is not None else torch.empty(M, N, dtype=torch.float32, device=A.device)
    ws = workspace
    if nb and (ws is None or ws.numel() * ws.element_size() < nb):
        ws = torch.empty(nb // 4, dtype=torch.float32, device=A.device)
    call('ck_gemm', _ptr(A), _ptr(B), _ptr(C), _ptr(bias), M, N, K, K, N if b_kn else K, N, 1 if b_kn else 0,
         tile, split_k, _ptr(ws) if nb else None, nb, _stream())
    return C


def gemm_epi(A, W, bias, epi, out, tile=0, split_k=0):
    """Fused-epilogue GEMM: A f16 [M, K], W f16 [N, K]; epi 1..4 (see chestnut.h)."""
    _need(A, torch.float16, 'A')
    _need(W, torch.float16, 'W')
    M, K = A.shape
    N = W.shape[0]
    tile, split_k, nb = gemm_workspace(M, N, K, False, tile, split_k)
    ws = torch.empty(max(nb // 4, 1), dtype=torch.float32, device=A.device)
    call('ck_gemm_epi', _ptr(A), _ptr(W), _ptr(out), _ptr(bias), M, N, K, K, K, N, epi, tile, split_k,
         _ptr(ws) if nb else None, nb, _stream())
    return out


def wmma_rdna4(fa, fb, fc):
    """RDNA4 WMMA fragments u16 [n,32,8] x2 + f32 [n,32,8] -> f32 [n,32,8]."""
    for t, dt, n in ((fa, torch.int16, 'fragA'), (fb, torch.int16, 'fragB'), (fc, torch.float32, 'fragC')):
        _need(t, dt, n)
    n = fa.shape[0]
    fd = torch.empty_like(fc)
    call('ck_wmma_rdna4', _ptr(fa), _ptr(fb), _ptr(fc), _ptr(fd), n, _stream())
    return fd


def mfma_kat(variant, A, B):
    _need(A, torch.int16, 'A')
    _need(B, torch.int16, 'B')
    M, N = (16, 16) if variant == 0 else (32, 32)
    D = torch.empty(M, N, dtype=torch.float32, device=A.device)
    call('ck_mfma_kat', variant, _ptr(A), _ptr(B), _ptr(D), _stream())
    return D


def pack_yuv(Y, U, V):
    for t, n in ((Y, 'Y'), (U, 'U'), (V, 'V')):
        _need(t, torch.uint8, n)
    H, W = Y.shape
    out = torch.empty(6, H // 2, W // 2, dtype=torch.uint8, device=Y.device)
    call('ck_pack_yuv', _ptr(Y), _ptr(U), _ptr(V), H, W, _ptr(out), _stream())
    return out


def frames_to_tensor(frame):
    _need(frame, torch.uint8, 'frame')
    H = frame.shape[0] * 2 // 3
    W = frame.shape[1]
    out = torch.empty(6, H // 2, W // 2, dtype=torch.uint8, device=frame.device)
    call('ck_frames_to_tensor', _ptr(frame), H, W, _ptr(out), _stream())
    return out


def img_gather(img, yx):
    """img [A, B, lanes] (any 1/2/4-byte dtype), yx int32 [n, 2] -> [n, lanes]."""
    if not img.is_contiguous():
        raise ValueError('img must be contiguous')
    _need(yx, torch.int32, 'yx')
    A, B, lanes = img.shape
    n = yx.shape[0]
    out = torch.empty(n, lanes, dtype=img.dtype, device=img.device)
    call('ck_img_gather', _ptr(img), A, B, lanes, img.element_size(), _ptr(yx), n, _ptr(out), _stream())
    return out


def attention(qk, vt, n_heads, head_dim):
    _need(qk, torch.float16, 'qk')
    _need(vt, torch.float16, 'vt')
    T = qk.shape[0]
    out = torch.empty(T, n_heads * head_dim, dtype=torch.float16, device=qk.device)
    call('ck_attention', _ptr(qk), _ptr(vt), _ptr(out), T, n_heads, head_dim, _stream())
    return out


def layernorm(x, g, b, eps=1e-5, out_f16=True):
    for t, n in ((x, 'x'), (g, 'g'), (b, 'b')):
        _need(t, torch.float32, n)
    rows, d = x.shape
    out = torch.empty(rows, d, dtype=torch.float16 if out_f16 else torch.float32, device=x.device)
    call('ck_layernorm', _ptr(x), _ptr(g), _ptr(b), _ptr(out), 1 if out_f16 else 0, rows, d, eps, _stream())
    return out


def warp_nv12(frame, big_frame, tfm, big_tfm, cam_w, cam_h, stride, y_height, model_w=512, model_h=256, out=None):
    """NV12 frames (u8 device buffers) + f32 [3,3] inverse transforms ->
    u8 [2, 6, model_h/2, model_w/2] (the engine's `warped`)."""
    for t, n in ((frame, 'frame'), (big_frame, 'big_frame')):
        _need(t, torch.uint8, n)
    for t, n in ((tfm, 'tfm'), (big_tfm, 'big_tfm')):
        _need(t, torch.float32, n)
    if frame.numel() != big_frame.numel() or tfm.numel() != 9 or big_tfm.numel() != 9:
        raise ValueError('frames must have the same size and transforms 9 floats')
    shape = (2, 6, model_h // 2, model_w // 2)
    if out is None:
        out = torch.empty(shape, dtype=torch.uint8, device=frame.device)
    else:
        _need(out, torch.uint8, 'out')
        if tuple(out.shape) != shape:
            raise ValueError(f'out must be uint8 {shape}')
    call('ck_warp_nv12', _ptr(frame), _ptr(big_frame), frame.numel(), _ptr(tfm), _ptr(big_tfm), cam_w, cam_h, stride,
         y_height, model_w, model_h, _ptr(out), _stream())
    return out
