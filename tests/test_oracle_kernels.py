"""Pins the oracle's GEMV / GEMM / WMMA restatements (CPU only).

Each check is independent of the formula it checks: brute-force loops,
closed forms (identity, permutation, linearity) or the reference's own KAT
vectors (tests/golden)."""
import numpy as np

from conftest import golden
from oracle import kernels as K


def test_gemv_bruteforce_small():
    rng = np.random.default_rng(0)
    W = rng.standard_normal((5, 24)).astype(np.float16)
    x = rng.uniform(-1, 1, 24).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    ref = [sum(float(W[r, k]) * float(x[k]) for k in range(24)) + float(b[r]) for r in range(5)]
    np.testing.assert_allclose(K.gemv(W, x, b), ref, rtol=1e-12, atol=1e-12)


def test_gemv_identity_and_linearity():
    rng = np.random.default_rng(1)
    x = rng.uniform(-1, 1, 64).astype(np.float32)
    I = np.eye(64, dtype=np.float16)
    np.testing.assert_array_equal(K.gemv(I, x), x.astype(np.float64))
    W = rng.standard_normal((7, 64)).astype(np.float16)
    y = rng.uniform(-1, 1, 64).astype(np.float32)
    lhs = K.gemv(W, (x.astype(np.float64) + y).astype(np.float32))
    # exact in float64 up to the f32 rounding of x + y
    xy = (x.astype(np.float64) + y.astype(np.float64)).astype(np.float32)
    np.testing.assert_allclose(lhs, K.gemv(W, xy), rtol=0, atol=0)
    np.testing.assert_allclose(K.gemv(W, x) + K.gemv(W, y), W.astype(np.float64) @ (x.astype(np.float64) + y),
                               rtol=1e-12, atol=1e-12)


def test_gemv_gelu_closed_form():
    W = np.eye(4, dtype=np.float16)
    x = np.array([0.0, 1.0, -1.0, 3.0], np.float32)
    g = K.gemv(W, x, act='gelu')
    assert g[0] == 0.0
    # gelu(x) - gelu(-x) = x for the tanh form
    assert abs((g[1] - g[2]) - 1.0) < 1e-12
    assert abs(g[3] - 3.0 * 0.5 * (1 + np.tanh(np.sqrt(2 / np.pi) * (3 + 0.044715 * 27)))) < 1e-12


def test_gelu_published_values_and_library():
    """The tanh form against values published for it (Hendrycks & Gimpel's
    approximation: gelu(1) = 0.841192, gelu(-1) = -0.158808, gelu(2) =
    1.954598) and against torch's own tanh-approximate GELU in float64; the
    erf form differs at x = 1 by 1.5e-4, so an erf GELU, a dropped cubic term
    or a wrong constant fails here."""
    import torch
    x = np.array([1.0, -1.0, 2.0])
    np.testing.assert_allclose(K.gelu(x), [0.841192, -0.158808, 1.954598], atol=1e-6)
    from math import erf, sqrt
    assert abs(K.gelu(np.array([1.0]))[0] - 0.5 * (1 + erf(1 / sqrt(2)))) > 1e-4
    grid = np.linspace(-8, 8, 4001)
    ref = torch.nn.functional.gelu(torch.from_numpy(grid), approximate='tanh').numpy()
    np.testing.assert_allclose(K.gelu(grid), ref, rtol=0, atol=1e-14)


def test_gemm_bruteforce_and_layouts():
    rng = np.random.default_rng(2)
    A = rng.standard_normal((4, 4)).astype(np.float16)
    B = rng.standard_normal((4, 4)).astype(np.float16)
    ref = np.array([[sum(float(A[i, k]) * float(B[k, j]) for k in range(4)) for j in range(4)] for i in range(4)])
    np.testing.assert_allclose(K.gemm(A, B), ref, rtol=1e-12)
    np.testing.assert_allclose(K.gemm(A, np.ascontiguousarray(B.T), transB=True), ref, rtol=1e-12)
    P = np.eye(4, dtype=np.float16)[[2, 0, 3, 1]]
    np.testing.assert_array_equal(K.gemm(P, B), B.astype(np.float64)[[2, 0, 3, 1]])


def test_kchain_matches_exact_within_sequential_bound():
    rng = np.random.default_rng(3)
    M, Kd, N = 8, 256, 8
    A = (rng.standard_normal((M, Kd)) / 16).astype(np.float16)
    B = (rng.standard_normal((Kd, N)) / 16).astype(np.float16)
    exact = K.gemm(A, B)
    chain = K.gemm_kchain16(A, B)
    scale = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    # sequential f32 summation: |err| <= K * 2^-24 * sum|a b|
    assert np.all(np.abs(chain - exact) <= Kd * 2.0 ** -24 * scale)
    assert not np.array_equal(chain.astype(np.float64), exact)   # really an f32 chain


def test_kchain_is_wmma_chain():
    """The 16-wide K chain equals chaining the oracle's WMMA through C."""
    rng = np.random.default_rng(4)
    A = rng.standard_normal((16, 32)).astype(np.float16)
    B = rng.standard_normal((32, 16)).astype(np.float16)
    C = np.zeros((16, 16), np.float32)
    for ks in range(2):
        fa, fb, fc = K.rdna4_fragments_from_matrix(A[:, 16 * ks:16 * ks + 16], B[16 * ks:16 * ks + 16], C)
        fd = K.wmma_rdna4(fa, fb, fc)
        for lane in range(32):
            for e in range(8):
                C[(lane // 16) * 8 + e, lane % 16] = fd[lane, e]
    np.testing.assert_array_equal(C, K.gemm_kchain16(A, B))


def test_rdna4_map_is_a_bijection():
    seen = set()
    for lane in range(32):
        for j in range(8):
            seen.add((lane % 16, K.rdna4_k(lane, j)))
    assert seen == {(r, k) for r in range(16) for k in range(16)}


def test_wmma_consumer_kat_golden():
    """consumer_probe.py's vector: bits lane*8+j+1 in both A and B."""
    z = golden('wmma_consumer_kat.npz')
    D = K.wmma_rdna4(z['fragA'], z['fragB'], z['fragC'])
    ref = z['Dfrag']
    assert np.max(np.abs(D - ref) / np.maximum(np.abs(ref), 1e-300)) < 1e-5
    A, B = K.rdna4_unpack(z['fragA'], z['fragB'])
    np.testing.assert_array_equal(A @ B, z['D'])


def test_wmma_rowcol_kat_golden():
    """mma_probe.py's row/column bit-pattern operands through the fragment map."""
    z = golden('mma_rowcol_kat.npz')
    A = z['A'].view(np.float16)
    B = z['B'].view(np.float16)
    fa, fb, fc = K.rdna4_fragments_from_matrix(A, B, np.zeros((16, 16), np.float32))
    D = K.wmma_rdna4(fa, fb, fc)
    Dm = np.zeros((16, 16))
    for lane in range(32):
        for e in range(8):
            Dm[(lane // 16) * 8 + e, lane % 16] = D[lane, e]
    ref = z['D']
    assert np.max(np.abs(Dm - ref) / np.maximum(np.abs(ref), 1e-300)) < 1e-5
    assert np.max(np.abs(Dm - ref)) <= 0.5   # the probe's own tolerance


def test_wmma_adds_c():
    rng = np.random.default_rng(5)
    A = np.zeros((16, 16), np.float16)
    B = np.zeros((16, 16), np.float16)
    C = rng.standard_normal((16, 16)).astype(np.float32)
    fa, fb, fc = K.rdna4_fragments_from_matrix(A, B, C)
    D = K.wmma_rdna4(fa, fb, fc)
    np.testing.assert_array_equal(D, fc)
