"""ck_gemm_noalloc (the allocation-free GEMM) through the C ABI: two calls in
a row, the second smaller, each bit-identical to ck_gemm with a caller
workspace (the same kernels and split order), plus the oracle within the GEMM
bound; a GEMM whose workspace exceeds the static scratch is rejected before
any launch."""
import ctypes

import numpy as np
import pytest

from chestnut import _lib
from oracle import kernels as OK

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def _p(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ws_bytes(M, N, K, b_kn, tile, split):
    t, s, nb = ctypes.c_int(tile), ctypes.c_int(split), ctypes.c_size_t()
    _lib.call('ck_gemm_workspace', M, N, K, b_kn, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    return t.value, s.value, nb.value


def _case(torch, M, N, K, b_kn, tile, split, seed, with_bias):
    rng = np.random.default_rng(seed)
    A = (rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float16)
    B = (rng.standard_normal((K, N) if b_kn else (N, K)) / 2).astype(np.float16)
    bias = rng.standard_normal(N).astype(np.float32) if with_bias else None
    Ad, Bd = torch.from_numpy(A).cuda(), torch.from_numpy(B).cuda()
    bd = torch.from_numpy(bias).cuda() if with_bias else None
    ldb = N if b_kn else K
    # the existing entry point, with a caller workspace
    t, s, nb = _ws_bytes(M, N, K, b_kn, tile, split)
    ws = torch.empty(max(nb // 4, 1), dtype=torch.float32, device='cuda')
    C_ref = torch.full((M, N), float('nan'), dtype=torch.float32, device='cuda')
    _lib.call('ck_gemm', _p(Ad), _p(Bd), _p(C_ref), _p(bd), M, N, K, K, ldb, N, b_kn, tile, split,
              _p(ws) if nb else None, nb, _stream(torch))
    # the allocation-free one
    C = torch.full((M, N), float('nan'), dtype=torch.float32, device='cuda')
    _lib.call('ck_gemm_noalloc', _p(Ad), _p(Bd), _p(C), _p(bd), M, N, K, K, ldb, N, b_kn, tile, split,
              _stream(torch))
    torch.cuda.synchronize()
    got, ref = C.cpu().numpy(), C_ref.cpu().numpy()
    return A, B, bias, got, ref, (t, s, nb)


def test_noalloc_gemm_two_calls_match_ck_gemm(gpu):
    torch = gpu
    # 1: BASELINE config 1 (1024 x 6144 x 1024, [K][N] B): tile 2, split 2,
    #    8 MiB of partials in the scratch
    print('[noalloc] call 1: 1024x1024x6144 b_kn', flush=True)
    A, B, _, got, ref, (t, s, nb) = _case(torch, 1024, 1024, 6144, 1, 0, 0, 1, False)
    assert s > 1 and nb > 0, 'the first case must use the scratch'
    np.testing.assert_array_equal(got, ref)
    exact = OK.gemm(A, B)
    bound = (6144 // 16 + 32) * U * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))
    assert np.all(np.abs(got - exact) <= bound)
    # 2: smaller, [N][K] B, bias, split 2 -- reuses the scratch the first call left
    print('[noalloc] call 2: 256x384x1024 nk split 2 bias', flush=True)
    A, B, bias, got, ref, (t, s, nb) = _case(torch, 256, 384, 1024, 0, 0, 2, 2, True)
    assert s == 2 and nb > 0
    np.testing.assert_array_equal(got, ref)
    exact = OK.gemm(A, B, transB=True) + bias
    bound = (1024 // 16 + 32) * U * ((np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)).T) + np.abs(bias))
    assert np.all(np.abs(got - exact) <= bound)


def test_noalloc_gemm_rejects_workspace_above_scratch(gpu):
    torch = gpu
    M, N, K = 2048, 2048, 8192
    t, s, nb = _ws_bytes(M, N, K, 0, 1, 8)
    assert nb > (32 << 20)
    A = torch.zeros(M, K, dtype=torch.float16, device='cuda')
    B = torch.zeros(N, K, dtype=torch.float16, device='cuda')
    C = torch.zeros(M, N, dtype=torch.float32, device='cuda')
    with pytest.raises(RuntimeError, match='static scratch'):
        _lib.call('ck_gemm_noalloc', _p(A), _p(B), _p(C), None, M, N, K, K, K, N, 0, 1, 8, _stream(torch))
    # nothing ran: C still zero
    assert not C.any().item()


def test_noalloc_gemm_under_graph_capture(gpu):
    """ck_gemm_noalloc captured into a graph (torch.cuda.graph, the current
    stream being the capture stream) and replayed three times: every replay
    is bit-identical to the eager call, with an eager call on another shape
    between the replays overwriting the shared scratch, so a replay reads
    only what it wrote itself."""
    torch = gpu
    rng = np.random.default_rng(5)
    M, N, K = 1024, 1024, 6144
    A = torch.from_numpy((rng.standard_normal((M, K)) / np.sqrt(K)).astype(np.float16)).cuda()
    B = torch.from_numpy((rng.standard_normal((K, N)) / 2).astype(np.float16)).cuda()
    C_eager = torch.full((M, N), float('nan'), dtype=torch.float32, device='cuda')
    print('[noalloc] graph: eager call (looks up the scratch address)', flush=True)
    _lib.call('ck_gemm_noalloc', _p(A), _p(B), _p(C_eager), None, M, N, K, K, N, N, 1, 0, 0, _stream(torch))
    torch.cuda.synchronize()
    A2 = torch.from_numpy((rng.standard_normal((256, 1024)) / 32).astype(np.float16)).cuda()
    B2 = torch.from_numpy((rng.standard_normal((384, 1024)) / 2).astype(np.float16)).cuda()
    C2 = torch.empty(256, 384, dtype=torch.float32, device='cuda')
    C = torch.full((M, N), float('nan'), dtype=torch.float32, device='cuda')
    g = torch.cuda.CUDAGraph()
    print('[noalloc] graph: capture', flush=True)
    with torch.cuda.graph(g):
        _lib.call('ck_gemm_noalloc', _p(A), _p(B), _p(C), None, M, N, K, K, N, N, 1, 0, 0, _stream(torch))
    torch.cuda.synchronize()
    ref = C_eager.cpu().numpy()
    for r in range(3):
        C.fill_(float('nan'))
        _lib.call('ck_gemm_noalloc', _p(A2), _p(B2), _p(C2), None, 256, 384, 1024, 1024, 1024, 384, 0, 0, 2,
                  _stream(torch))
        torch.cuda.synchronize()
        print(f'[noalloc] graph: replay {r}', flush=True)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(C.cpu().numpy(), ref)
