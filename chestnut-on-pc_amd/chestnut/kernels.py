"""Per-kernel entry points on torch device tensors (probe / bench harness).

torch provides device memory and the current stream only; every computation
is a call into libchestnut.so.  The native side receives raw pointers plus
sizes, so every tensor argument is validated here first -- dtype, shape
against the sizes derived from the operands, contiguity, and that all of
them live on the current CUDA device -- and a mismatch raises ValueError
before anything is launched.  The native entry points then check sizes and
alignment again.  Shapes are checked before the device, so the checks run
(and are tested) without a GPU.
"""
import ctypes

import torch

from ._lib import call


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _check(t, dtype, name, shape=None):
    """dtype, exact shape (None entries are free) and contiguity of one tensor."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f'{name} must be a torch tensor')
    if t.dtype != dtype:
        raise ValueError(f'{name} must be {dtype}, got {t.dtype}')
    if shape is not None:
        ok = t.dim() == len(shape) and all(s is None or int(a) == int(s) for a, s in zip(t.shape, shape))
        if not ok:
            want = tuple('*' if s is None else int(s) for s in shape)
            raise ValueError(f'{name} must have shape {want}, got {tuple(t.shape)}')
    if not t.is_contiguous():
        raise ValueError(f'{name} must be contiguous')


def _validate(*args):
    """args: (tensor or None, dtype, name[, shape]).  Every present tensor is
    checked for dtype, shape and contiguity, then all of them for placement
    on the current CUDA device."""
    present = [a for a in args if a[0] is not None]
    for a in present:
        _check(*a)
    for a in present:
        t, name = a[0], a[2]
        if not t.is_cuda:
            raise ValueError(f'{name} must be a CUDA tensor')
        if t.device.index != torch.cuda.current_device():
            raise ValueError(f'{name} is on {t.device}, not the current device cuda:{torch.cuda.current_device()}')


def gemv(W, x, bias=None, act=0, rows_per_wg=0, out=None):
    """y = act(W @ x + bias): W f16 [rows, K], x f32 [K] -> f32 [rows]."""
    if W.dim() != 2:
        raise ValueError('W must be 2-D [rows, K]')
    rows, K = W.shape
    if act not in (0, 1):
        raise ValueError('act must be 0 (none) or 1 (gelu)')
    _validate((W, torch.float16, 'W'), (x, torch.float32, 'x', (K,)), (bias, torch.float32, 'bias', (rows,)),
              (out, torch.float32, 'out', (rows,)))
    y = out if out is not None else torch.empty(rows, dtype=torch.float32, device=W.device)
    call('ck_gemv', _ptr(W), _ptr(x), _ptr(bias), _ptr(y), rows, K, K, act, rows_per_wg, _stream())
    return y


def gemm_workspace(M, N, K, b_kn, tile=0, split_k=0):
    t, s, nb = ctypes.c_int(tile), ctypes.c_int(split_k), ctypes.c_size_t()
    call('ck_gemm_workspace', M, N, K, 1 if b_kn else 0, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    return t.value, s.value, nb.value


def _workspace(ws, nb, device):
    """The caller's f32 workspace if it holds nb bytes, else a new one."""
    if not nb:
        return None
    if ws is not None:
        _validate((ws, torch.float32, 'workspace'))
        if ws.numel() * 4 >= nb:
            return ws
    return torch.empty(nb // 4, dtype=torch.float32, device=device)


def gemm(A, B, b_kn=True, bias=None, tile=0, split_k=0, out=None, workspace=None):
    """C f32 = A @ B (+ bias): A f16 [M, K]; B f16 [K, N] (b_kn) or [N, K]."""
    if A.dim() != 2 or B.dim() != 2:
        raise ValueError('A and B must be 2-D')
    M, K = A.shape
    N = B.shape[1] if b_kn else B.shape[0]
    _validate((A, torch.float16, 'A'), (B, torch.float16, 'B', (K, N) if b_kn else (N, K)),
              (bias, torch.float32, 'bias', (N,)), (out, torch.float32, 'out', (M, N)))
    tile, split_k, nb = gemm_workspace(M, N, K, b_kn, tile, split_k)
    C = out if out is not None else torch.empty(M, N, dtype=torch.float32, device=A.device)
    ws = _workspace(workspace, nb, A.device)
    call('ck_gemm', _ptr(A), _ptr(B), _ptr(C), _ptr(bias), M, N, K, K, N if b_kn else K, N, 1 if b_kn else 0,
         tile, split_k, _ptr(ws), nb, _stream())
    return C


_EPI_OUT = {1: torch.float16, 2: torch.float16, 3: torch.float16, 4: torch.float32}


def gemm_epi(A, W, bias, epi, out, tile=0, split_k=0):
    """Fused-epilogue GEMM: A f16 [M, K], W f16 [N, K], bias f32 [N] or None;
    epi 1 f16(acc+bias), 2 f16(relu), 3 f16(gelu) -> out f16 [M, N];
    epi 4 out f32 [M, N] += acc + bias."""
    if epi not in _EPI_OUT:
        raise ValueError('epi must be 1..4')
    if A.dim() != 2 or W.dim() != 2:
        raise ValueError('A and W must be 2-D')
    M, K = A.shape
    N = W.shape[0]
    if out is None:
        raise ValueError('out is required')
    _validate((A, torch.float16, 'A'), (W, torch.float16, 'W', (N, K)), (bias, torch.float32, 'bias', (N,)),
              (out, _EPI_OUT[epi], 'out', (M, N)))
    tile, split_k, nb = gemm_workspace(M, N, K, False, tile, split_k)
    ws = _workspace(None, nb, A.device)
    call('ck_gemm_epi', _ptr(A), _ptr(W), _ptr(out), _ptr(bias), M, N, K, K, K, N, epi, tile, split_k,
         _ptr(ws), nb, _stream())
    return out


def wmma_rdna4(fa, fb, fc):
    """RDNA4 WMMA fragments u16 [n,32,8] x2 + f32 [n,32,8] -> f32 [n,32,8]."""
    if fa.dim() != 3:
        raise ValueError('fragA must be [n, 32, 8]')
    n = fa.shape[0]
    _validate((fa, torch.int16, 'fragA', (n, 32, 8)), (fb, torch.int16, 'fragB', (n, 32, 8)),
              (fc, torch.float32, 'fragC', (n, 32, 8)))
    fd = torch.empty_like(fc)
    call('ck_wmma_rdna4', _ptr(fa), _ptr(fb), _ptr(fc), _ptr(fd), n, _stream())
    return fd


def mfma_kat(variant, A, B):
    """One MFMA on row-major operands: variant 0 A [16,32] B [32,16];
    variant 1 A [32,16] B [16,32]."""
    if variant not in (0, 1):
        raise ValueError('variant must be 0 (16x16x32) or 1 (32x32x16)')
    M, N, Kk = (16, 16, 32) if variant == 0 else (32, 32, 16)
    _validate((A, torch.int16, 'A', (M, Kk)), (B, torch.int16, 'B', (Kk, N)))
    D = torch.empty(M, N, dtype=torch.float32, device=A.device)
    call('ck_mfma_kat', variant, _ptr(A), _ptr(B), _ptr(D), _stream())
    return D


def pack_yuv(Y, U, V):
    """Full-resolution Y, U, V planes u8 [H, W] -> u8 [6, H/2, W/2]."""
    if Y.dim() != 2 or Y.shape[0] % 2 or Y.shape[1] % 2:
        raise ValueError('Y must be u8 [H, W] with H and W even')
    H, W = Y.shape
    _validate((Y, torch.uint8, 'Y', (H, W)), (U, torch.uint8, 'U', (H, W)), (V, torch.uint8, 'V', (H, W)))
    out = torch.empty(6, H // 2, W // 2, dtype=torch.uint8, device=Y.device)
    call('ck_pack_yuv', _ptr(Y), _ptr(U), _ptr(V), H, W, _ptr(out), _stream())
    return out


def frames_to_tensor(frame):
    """I420 frame u8 [H*3/2, W] -> u8 [6, H/2, W/2]."""
    if frame.dim() != 2 or frame.shape[0] % 6 or frame.shape[1] % 2:
        raise ValueError('frame must be u8 [H*3/2, W] with H a multiple of 4 and W even')
    _validate((frame, torch.uint8, 'frame'))
    H = frame.shape[0] * 2 // 3
    W = frame.shape[1]
    out = torch.empty(6, H // 2, W // 2, dtype=torch.uint8, device=frame.device)
    call('ck_frames_to_tensor', _ptr(frame), H, W, _ptr(out), _stream())
    return out


def img_gather(img, yx):
    """img [A, B, lanes] (any 1/2/4-byte dtype), yx int32 [n, 2] -> [n, lanes]."""
    if img.dim() != 3 or img.element_size() not in (1, 2, 4):
        raise ValueError('img must be [A, B, lanes] of a 1-, 2- or 4-byte dtype')
    if yx.dim() != 2:
        raise ValueError('yx must be int32 [n, 2]')
    _validate((img, img.dtype, 'img'), (yx, torch.int32, 'yx', (yx.shape[0], 2)))
    A, B, lanes = img.shape
    n = yx.shape[0]
    out = torch.empty(n, lanes, dtype=img.dtype, device=img.device)
    call('ck_img_gather', _ptr(img), A, B, lanes, img.element_size(), _ptr(yx), n, _ptr(out), _stream())
    return out


def attention(qk, vt, n_heads, head_dim):
    """qk f16 [T, 2d] (Q | K), vt f16 [d, T] -> f16 [T, d], d = n_heads * head_dim."""
    d = n_heads * head_dim
    if qk.dim() != 2:
        raise ValueError('qk must be f16 [T, 2d]')
    T = qk.shape[0]
    _validate((qk, torch.float16, 'qk', (T, 2 * d)), (vt, torch.float16, 'vt', (d, T)))
    out = torch.empty(T, d, dtype=torch.float16, device=qk.device)
    call('ck_attention', _ptr(qk), _ptr(vt), _ptr(out), T, n_heads, head_dim, _stream())
    return out


def layernorm(x, g, b, eps=1e-5, out_f16=True):
    """Row LayerNorm of x f32 [rows, d] with g, b f32 [d] -> f16 or f32 [rows, d]."""
    if x.dim() != 2:
        raise ValueError('x must be f32 [rows, d]')
    rows, d = x.shape
    _validate((x, torch.float32, 'x'), (g, torch.float32, 'g', (d,)), (b, torch.float32, 'b', (d,)))
    out = torch.empty(rows, d, dtype=torch.float16 if out_f16 else torch.float32, device=x.device)
    call('ck_layernorm', _ptr(x), _ptr(g), _ptr(b), _ptr(out), 1 if out_f16 else 0, rows, d, eps, _stream())
    return out


def warp_nv12(frame, big_frame, tfm, big_tfm, cam_w, cam_h, stride, y_height, model_w=512, model_h=256, out=None,
              division='ieee'):
    """NV12 frames (u8 device buffers) + f32 [3,3] inverse transforms ->
    u8 [2, 6, model_h/2, model_w/2] (the engine's `warped`).  division:
    'ieee' (src_x / src_w) or 'rcp' (src_x * (1 / src_w)), as
    oracle.warp's `div`."""
    if division not in ('ieee', 'rcp'):
        raise ValueError("division must be 'ieee' or 'rcp'")
    nb = stride * y_height + (cam_h // 2) * stride
    for t, n in ((frame, 'frame'), (big_frame, 'big_frame')):
        if t.numel() != nb:
            raise ValueError(f'{n} must hold {nb} bytes of NV12 (stride {stride}, y_height {y_height}), '
                             f'got {t.numel()}')
    for t, n in ((tfm, 'tfm'), (big_tfm, 'big_tfm')):
        if t.numel() != 9:
            raise ValueError(f'{n} must be 3x3')
    shape = (2, 6, model_h // 2, model_w // 2)
    _validate((frame, torch.uint8, 'frame'), (big_frame, torch.uint8, 'big_frame'), (tfm, torch.float32, 'tfm'),
              (big_tfm, torch.float32, 'big_tfm'), (out, torch.uint8, 'out', shape))
    if out is None:
        out = torch.empty(shape, dtype=torch.uint8, device=frame.device)
    call('ck_warp_nv12', _ptr(frame), _ptr(big_frame), frame.numel(), _ptr(tfm), _ptr(big_tfm), cam_w, cam_h, stride,
         y_height, model_w, model_h, 1 if division == 'rcp' else 0, _ptr(out), _stream())
    return out
