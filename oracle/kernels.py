"""Oracle restatements of the reduction / matrix kernels on the hot path.

Test infrastructure only (see oracle/__init__.py).
"""
import numpy as np


# ---------------------------------------------------------------------------
# serial reduce r_32_32_3_12288_32 -> GEMV
# ---------------------------------------------------------------------------
def gemv(W16, x32, bias=None, act=None):
    """out[r] = sum_k W[r,k] * x[k] (+ bias[r]), evaluated in float64.

    Restates the reduction of `r_32_32_3_12288_32` (run_pinned2.py:989-1066,
    alu_opt.py:1-12): a 12288-long dot product per output with f32 inputs,
    which the reference computes serially and `_warp_split_ptx` reassociates
    into W strided partial sums (run_pinned2.py:1031-1047).  The exact value
    (float64 of the f16-rounded weights and f32 activations) is the target
    every summation order approximates.

    act: None or 'gelu' (tanh form, applied after the bias, in float64).
    Returns float64; callers round as the device path does.
    Pinned by: brute-force loop on small shapes; linearity in x; identity
    matrix reproduces x (tests/test_oracle_kernels.py).
    """
    W = np.asarray(W16, dtype=np.float16).astype(np.float64)
    x = np.asarray(x32, dtype=np.float32).astype(np.float64)
    y = W @ x
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float32).astype(np.float64)
    if act == 'gelu':
        y = gelu(y)
    elif act is not None:
        raise ValueError(f'unknown act {act!r}')
    return y


def gemv_abs(W16, x32):
    """sum_k |W[r,k] * x[k]| in float64: the scale a summation-order error
    bound is stated against."""
    W = np.abs(np.asarray(W16, dtype=np.float16).astype(np.float64))
    x = np.abs(np.asarray(x32, dtype=np.float32).astype(np.float64))
    return W @ x


# ---------------------------------------------------------------------------
# WMMA attention/projection GEMMs (r_6_2, r_2_24, r_12_32_4, r_48_32_4)
# ---------------------------------------------------------------------------
def gemm(A16, B16, transB=False):
    """C = A @ B with f16 inputs, evaluated exactly in float64.

    The GEMM the WMMA kernels compute: f16 operands, f32 accumulation, stores
    after the K loop (NOTES.md:87-91; run_pinned2.py:866-872).  B is [K,N], or
    [N,K] when transB (the weight layout of the model's projections).
    Pinned by: K-chained fp32 emulation agrees within f32 accumulation error;
    identity / permutation matrices; brute force on 4x4x4.
    """
    A = np.asarray(A16, dtype=np.float16).astype(np.float64)
    B = np.asarray(B16, dtype=np.float16).astype(np.float64)
    return A @ (B.T if transB else B)


def gemm_kchain16(A16, B16):
    """C f32 = A @ B accumulated as the WMMA FFMA consumer does it.

    The reference's FFMA consumer computes each 16x16x16 WMMA as a chain of
    16 fused multiply-adds per output, k = 0..15, starting from the running
    C fragment (run_pinned2.py:183-191), and the GEMM kernels chain WMMAs
    along K in 16-wide steps through C (config 1: 384 trips).  Net effect:
    one sequential f32 FMA chain over k = 0..K-1.  The product of two f16
    values is exact in f32 (11+11 significand bits <= 24), so
    round(c + a*b) computed as two numpy f32 ops equals fma(a, b, c).
    Pinned by: agreement with `gemm` within the sequential-sum error bound,
    and with the FFMA chain of `wmma_rdna4` per 16-step.
    """
    A = np.asarray(A16, dtype=np.float16).astype(np.float32)
    B = np.asarray(B16, dtype=np.float16).astype(np.float32)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    C = np.zeros((M, N), np.float32)
    for k in range(K):
        C += A[:, k:k + 1] * B[k:k + 1, :]
    return C


# RDNA4 wave32 WMMA fragment map ((16,16,16), half, 'AMD', 32):
# run_pinned2.py:106-117 and consumer_probe.py:14-19.
def rdna4_k(lane, j):
    """K index held by element j (0..7) of `lane` (0..31) in an A/B fragment.

    lane < 16: j = 0..3 -> k = j,     j = 4..7 -> k = j + 4
    lane >= 16: j = 0..3 -> k = j + 4, j = 4..7 -> k = j + 8
    (consumer_probe.py:14-19; equivalently k = jA^-1 with
    jA(k) = k - [0,4,4,8][k//4], g(k) = (k//4)%2, run_pinned2.py:115-117).
    """
    if j < 4:
        return j if lane < 16 else j + 4
    return j + 4 if lane < 16 else j + 8


def rdna4_unpack(fragA, fragB):
    """Per-lane A/B fragments (u16 bit patterns [32,8]) -> A[16,16], B[16,16]
    as float64 values (A[row][k] from lane row%16 + 16*g(k); B[k][col] from
    lane col%16 + 16*g(k); run_pinned2.py:110-113)."""
    fa = np.asarray(fragA, dtype=np.uint16).view(np.float16).astype(np.float64)
    fb = np.asarray(fragB, dtype=np.uint16).view(np.float16).astype(np.float64)
    A = np.zeros((16, 16))
    B = np.zeros((16, 16))
    for lane in range(32):
        for j in range(8):
            k = rdna4_k(lane, j)
            A[lane % 16, k] = fa[lane, j]
            B[k, lane % 16] = fb[lane, j]
    return A, B


def wmma_rdna4(fragA, fragB, fragC):
    """D fragment [32,8] f32 of one WMMA uop, FFMA-consumer order.

    D[m][n] = fma chain over k = 0..15 starting from C (run_pinned2.py:183-191);
    lane element e of D is D[(lane//16)*8 + e][lane%16] (run_pinned2.py:114).
    """
    A, B = rdna4_unpack(fragA, fragB)
    A32 = A.astype(np.float32)
    B32 = B.astype(np.float32)
    C = np.asarray(fragC, dtype=np.float32)
    D = np.zeros((32, 8), np.float32)
    for lane in range(32):
        for e in range(8):
            m, n = (lane // 16) * 8 + e, lane % 16
            acc = np.float32(C[lane, e])
            for k in range(16):
                acc = np.float32(acc + A32[m, k] * B32[k, n])
            D[lane, e] = acc
    return D


def rdna4_fragments_from_matrix(A, B, C):
    """Inverse of the fragment map: A[16,16], B[16,16] (f16) and C[16,16] f32
    -> per-lane fragments (u16 [32,8], u16 [32,8], f32 [32,8])."""
    A = np.asarray(A, np.float16)
    B = np.asarray(B, np.float16)
    fa = np.zeros((32, 8), np.float16)
    fb = np.zeros((32, 8), np.float16)
    fc = np.zeros((32, 8), np.float32)
    for lane in range(32):
        for j in range(8):
            k = rdna4_k(lane, j)
            fa[lane, j] = A[lane % 16, k]
            fb[lane, j] = B[k, lane % 16]
        for e in range(8):
            fc[lane, e] = C[(lane // 16) * 8 + e, lane % 16]
    return fa.view(np.uint16), fb.view(np.uint16), fc


# ---------------------------------------------------------------------------
# elementwise helpers shared with the model oracle
# ---------------------------------------------------------------------------
GELU_C = np.sqrt(2.0 / np.pi)


def gelu(x):
    """tanh-form GELU: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    x = np.asarray(x)
    dt = x.dtype if x.dtype in (np.float32, np.float64) else np.float64
    c = dt.type(GELU_C)
    return (dt.type(0.5) * x * (dt.type(1.0) + np.tanh(c * (x + dt.type(0.044715) * x * x * x)))).astype(dt)
