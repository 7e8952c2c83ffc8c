"""GPU parity of the per-kernel entry points against the oracle.

Bit-exact for integer / byte / index work; floating point against stated
bounds derived from f32 summation error (|err| <= depth * 2^-24 * sum|terms|)
plus the north-star bound for f16-input GEMMs (max-abs <= 1e-2 relative)."""
import numpy as np
import pytest

from conftest import golden
from oracle import image as OI
from oracle import kernels as OK
from oracle import model as OM
from oracle import pack as OP

pytestmark = pytest.mark.gpu
U = 2.0 ** -24


def dev(torch, a):
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return torch.from_numpy(a.view(np.int16)).cuda().view(torch.float16)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16)).cuda()
    return torch.from_numpy(a).cuda()


def host(t):
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------- KATs ----
def test_mfma_layout_kat(gpu):
    from chestnut import kernels as K
    rng = np.random.default_rng(0)
    for variant, (M, Kd, N) in ((0, (16, 32, 16)), (1, (32, 16, 32))):
        print(f'[kat] mfma variant {variant}', flush=True)
        A = rng.standard_normal((M, Kd)).astype(np.float16)
        B = rng.standard_normal((Kd, N)).astype(np.float16)
        D = host(K.mfma_kat(variant, dev(gpu, A.view(np.uint16)), dev(gpu, B.view(np.uint16))))
        ref = A.astype(np.float64) @ B.astype(np.float64)
        scale = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
        assert np.all(np.abs(D - ref) <= (Kd + 2) * U * scale), 'MFMA operand layout mismatch'


def test_wmma_consumer_kat(gpu):
    """consumer_probe.py's KAT (bits lane*8+j+1) through the RDNA4 map on MFMA."""
    from chestnut import kernels as K
    z = golden('wmma_consumer_kat.npz')
    fd = host(K.wmma_rdna4(dev(gpu, z['fragA'][None]), dev(gpu, z['fragB'][None]), dev(gpu, z['fragC'][None])))[0]
    ref = z['Dfrag']
    # the probe's own criterion (consumer_probe.py:162-168) ...
    assert np.max(np.abs(fd - ref) / np.maximum(1.0, np.abs(ref))) <= 1e-5
    # ... and a relative one that the tiny subnormal-product values cannot pass by accident
    assert np.max(np.abs(fd - ref) / np.abs(ref)) <= 1e-5


def test_wmma_rowcol_and_random(gpu):
    from chestnut import kernels as K
    z = golden('mma_rowcol_kat.npz')
    rng = np.random.default_rng(1)
    mats = [(z['A'].view(np.float16), z['B'].view(np.float16), np.zeros((16, 16), np.float32))]
    for _ in range(7):
        mats.append((rng.standard_normal((16, 16)).astype(np.float16), rng.standard_normal((16, 16)).astype(np.float16),
                     rng.standard_normal((16, 16)).astype(np.float32)))
    fr = [OK.rdna4_fragments_from_matrix(*m) for m in mats]
    fa = np.stack([f[0] for f in fr])
    fb = np.stack([f[1] for f in fr])
    fc = np.stack([f[2] for f in fr])
    fd = host(K.wmma_rdna4(dev(gpu, fa), dev(gpu, fb), dev(gpu, fc)))
    for t in range(len(mats)):
        ref = OK.wmma_rdna4(fa[t], fb[t], fc[t])          # FFMA-consumer order
        A, B = OK.rdna4_unpack(fa[t], fb[t])
        scale = (np.abs(A) @ np.abs(B))
        sfrag = np.zeros((32, 8))
        for lane in range(32):
            for e in range(8):
                sfrag[lane, e] = scale[(lane // 16) * 8 + e, lane % 16] + abs(fc[t][lane, e])
        assert np.all(np.abs(fd[t] - ref) <= 36 * U * sfrag + 1e-30), f'tile {t}'
    Dm = np.zeros((16, 16))
    for lane in range(32):
        for e in range(8):
            Dm[(lane // 16) * 8 + e, lane % 16] = fd[0][lane, e]
    assert np.max(np.abs(Dm - z['D']) / np.abs(z['D'])) <= 1e-5


# ---------------------------------------------------------------- GEMV ----
def _gemv_bound(W, x, nstep):
    return (8 * nstep + 16) * U * OK.gemv_abs(W, x) + 1e-30


def test_gemv_config2_full_size(gpu):
    """W f16 [3072 x 12288] ~ N(0, 0.02), x f32 ~ U(-1, 1)."""
    from chestnut import kernels as K
    print('[gemv] config 2 3072x12288', flush=True)
    rng = np.random.default_rng(42)
    W = (rng.standard_normal((3072, 12288), dtype=np.float32) * 0.02).astype(np.float16)
    x = rng.uniform(-1, 1, 12288).astype(np.float32)
    Wd, xd = dev(gpu, W), dev(gpu, x)
    y = host(K.gemv(Wd, xd))
    ref = OK.gemv(W, x)
    assert np.all(np.abs(y - ref) <= _gemv_bound(W, x, 6))
    # deterministic, and independent of the row partition
    np.testing.assert_array_equal(host(K.gemv(Wd, xd)), y)
    for rpw in (4, 12, 64):
        np.testing.assert_array_equal(host(K.gemv(Wd, xd, rows_per_wg=rpw)), y)


@pytest.mark.parametrize('rows,Kd,act', [(1, 8, 0), (7, 3280, 0), (1536, 2048, 1), (1673, 512, 0), (5, 16384, 1),
                                         (37, 136, 1)])
def test_gemv_shapes_bias_act(gpu, rows, Kd, act):
    from chestnut import kernels as K
    rng = np.random.default_rng(rows + Kd)
    W = (rng.standard_normal((rows, Kd)) * 0.05).astype(np.float16)
    x = rng.uniform(-1, 1, Kd).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32)
    y = host(K.gemv(dev(gpu, W), dev(gpu, x), dev(gpu, b), act=act))
    ref = OK.gemv(W, x, b, act='gelu' if act else None)
    nstep = -(-Kd // 2048)
    bound = _gemv_bound(W, x, nstep) + 4 * U * np.abs(b)
    if act:
        bound = bound * 1.2 + 4 * U * np.abs(ref)
    assert np.all(np.abs(y - ref) <= bound)


@pytest.mark.parametrize('rows,Kd,act', [(1, 8, 0), (9, 136, 1), (1673, 512, 0)])
def test_gemv_wave_form_matches_workgroup_form(gpu, rows, Kd, act):
    """K <= 512 with the automatic row partition runs one wave per row; a
    pinned rows_per_wg runs the workgroup form.  The lane products and the
    wave sum are the same and the workgroup form's extra partials are exact
    zeros, so the two agree bit for bit."""
    from chestnut import kernels as K
    rng = np.random.default_rng(7 * rows + Kd)
    W = dev(gpu, (rng.standard_normal((rows, Kd)) * 0.05).astype(np.float16))
    x = dev(gpu, rng.uniform(-1, 1, Kd).astype(np.float32))
    b = dev(gpu, rng.standard_normal(rows).astype(np.float32))
    y = host(K.gemv(W, x, b, act=act))
    for rpw in (4, 8):
        np.testing.assert_array_equal(host(K.gemv(W, x, b, act=act, rows_per_wg=rpw)), y)


# ---------------------------------------------------------------- GEMM ----
def _gemm_check(C, A, B, transB=False, depth=None):
    ref = OK.gemm(A, B, transB)
    Bm = B.astype(np.float64).T if transB else B.astype(np.float64)
    scale = np.abs(A.astype(np.float64)) @ np.abs(Bm)
    Kd = A.shape[1]
    depth = depth or (Kd // 16 + 32)
    err = np.abs(C - ref)
    assert np.max(err) / np.max(np.abs(ref)) <= 1e-2
    assert np.all(err <= depth * U * scale + 1e-30), float(np.max(err / (scale + 1e-30)))
    return ref


def test_gemm_config1_full_size(gpu):
    """A f16 [1024 x 6144], B f16 [6144 x 1024] ~ N(0,1)/sqrt(6144), C f32."""
    from chestnut import kernels as K
    print('[gemm] config 1 1024x6144x1024', flush=True)
    rng = np.random.default_rng(42)
    A = (rng.standard_normal((1024, 6144), dtype=np.float32) / np.sqrt(6144)).astype(np.float16)
    B = (rng.standard_normal((6144, 1024), dtype=np.float32) / np.sqrt(6144)).astype(np.float16)
    Ad, Bd = dev(gpu, A), dev(gpu, B)
    C = host(K.gemm(Ad, Bd, b_kn=True))
    _gemm_check(C, A, B)
    np.testing.assert_array_equal(host(K.gemm(Ad, Bd, b_kn=True)), C)   # deterministic split-K
    C1 = host(K.gemm(Ad, Bd, b_kn=True, split_k=1))
    _gemm_check(C1, A, B)
    # same problem with B stored [N][K]
    Ct = host(K.gemm(Ad, dev(gpu, np.ascontiguousarray(B.T)), b_kn=False))
    _gemm_check(Ct, A, B)
    # the 128x64 tile at split 2, B loaded through registers (deterministic too)
    C2 = host(K.gemm(Ad, Bd, b_kn=True, tile=2, split_k=2))
    _gemm_check(C2, A, B)
    np.testing.assert_array_equal(host(K.gemm(Ad, Bd, b_kn=True, tile=2, split_k=2)), C2)


@pytest.mark.parametrize('b_kn,tile,M,N,Kd', [(True, 2, 1024, 1024, 6144), (False, 2, 1024, 1024, 6144),
                                              (True, 2, 300, 192, 768), (True, 1, 300, 384, 1024),
                                              (False, 1, 300, 520, 1024), (False, 2, 300, 520, 1024),
                                              (False, 3, 100, 200, 512), (False, 4, 100, 200, 256),
                                              (False, 4, 64, 128, 256), (True, 5, 100, 200, 512)])
@pytest.mark.parametrize('with_bias', [False, True])
def test_gemm_split2_equals_sum_of_halves(gpu, b_kn, tile, M, N, Kd, with_bias):
    """Split 2 with an f32 output is bit for bit (0 + p0) + p1 (+ bias), where
    p0 and p1 are the split-1 products of the two K halves on the same tile:
    what the split-K reduce computes, and what the in-kernel finish of the
    staged two-group tiles (2 with a [K][N] B; 2, 3, 4 with [N][K]) computes,
    whichever workgroup of a pair finishes last -- on every one of 10 launches
    (40 for the small shapes), with NaN in C and the partial planes before
    each (a partial read before its stores were visible shows up as NaN);
    ragged M and N."""
    from chestnut import kernels as K
    torch = gpu
    print(f'[gemm] split-2 halves b_kn={b_kn} tile={tile} {M}x{N}x{Kd} bias={with_bias}', flush=True)
    rng = np.random.default_rng(M + N + Kd + tile)
    A = (rng.standard_normal((M, Kd)) / 16).astype(np.float16)
    B = (rng.standard_normal((Kd, N) if b_kn else (N, Kd)) / 16).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32) if with_bias else None
    h = Kd // 2
    Bh = (B[:h], B[h:]) if b_kn else (B[:, :h], B[:, h:])
    p0 = host(K.gemm(dev(torch, A[:, :h]), dev(torch, Bh[0]), b_kn=b_kn, tile=tile, split_k=1))
    p1 = host(K.gemm(dev(torch, A[:, h:]), dev(torch, Bh[1]), b_kn=b_kn, tile=tile, split_k=1))
    want = (np.float32(0) + p0) + p1
    if with_bias:
        want = want + b
    Ad, Bd, bd = dev(torch, A), dev(torch, B), (dev(torch, b) if with_bias else None)
    C = torch.empty(M, N, device='cuda')
    _, _, nb = K.gemm_workspace(M, N, Kd, b_kn, tile, 2)
    ws = torch.empty(nb // 4, device='cuda')
    for r in range(10 if M * N > 200000 else 40):
        C.fill_(float('nan'))
        ws.fill_(float('nan'))
        K.gemm(Ad, Bd, b_kn=b_kn, bias=bd, tile=tile, split_k=2, out=C, workspace=ws)
        got = host(C)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f'launch {r}'


def test_gemm_split2_on_concurrent_streams(gpu):
    """Split-2 GEMMs in flight at once on two streams, each with its own
    workspace (NaN-filled) and, for the in-kernel finish, its own ticket
    slot: every result matches its single-stream value."""
    from chestnut import kernels as K
    torch = gpu
    rng = np.random.default_rng(5)
    M, N, Kd = 512, 512, 3072
    As = [dev(torch, (rng.standard_normal((M, Kd)) / 16).astype(np.float16)) for _ in range(2)]
    Bs = [dev(torch, (rng.standard_normal((Kd, N)) / 16).astype(np.float16)) for _ in range(2)]
    want = [host(K.gemm(As[i], Bs[i], b_kn=True, tile=2, split_k=2)) for i in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty(M, N, device='cuda') for _ in range(8)] for _ in range(2)]
    _, _, nb = K.gemm_workspace(M, N, Kd, True, 2, 2)
    wss = [[torch.full((nb // 4,), float('nan'), device='cuda') for _ in range(8)] for _ in range(2)]
    torch.cuda.synchronize()
    for r in range(8):
        for i in range(2):
            with torch.cuda.stream(streams[i]):
                K.gemm(As[i], Bs[i], b_kn=True, tile=2, split_k=2, out=outs[i][r], workspace=wss[i][r])
    torch.cuda.synchronize()
    for i in range(2):
        for r in range(8):
            assert np.array_equal(host(outs[i][r]), want[i]), f'stream {i} launch {r}'


@pytest.mark.parametrize('tile', [0, 1, 2, 4, 5, 9, 11, 13])
@pytest.mark.parametrize('M,N,Kd,split', [(100, 200, 320, 1), (300, 136, 1024, 2), (100, 256, 384, 1),
                                          (300, 384, 1024, 4), (64, 128, 256, 2), (300, 192, 768, 1),
                                          (64, 128, 1536, 2)])
def test_gemm_kn_paths(gpu, tile, M, N, Kd, split):
    """[K][N] B: with N a multiple of 128 the two-K-group 128x128 LDS-DMA
    tile (1, and 0 when it picks it) and the 8-wave 256x128 tile (9) stream
    it into LDS as it is and read their MFMA fragments transposed; the
    128x64 tile (2) with N a multiple of 64 and K per split a multiple of 384
    loads it through registers and writes it to LDS in the [N][K] layout;
    otherwise the LDS-DMA tiles (2, 4, 5, 9, ...) transpose it into the
    workspace first, and the register-staged tiles (11, 13) transpose it in
    registers; ragged M and N."""
    from chestnut import kernels as K
    rng = np.random.default_rng(M + N + tile)
    A = rng.standard_normal((M, Kd)).astype(np.float16)
    B = rng.standard_normal((Kd, N)).astype(np.float16)
    C = host(K.gemm(dev(gpu, A), dev(gpu, B), b_kn=True, tile=tile, split_k=split))
    _gemm_check(C, A, B)


def test_gemm_matches_kchain_semantics(gpu):
    """Against the reference's FFMA-chain accumulation (16-wide K steps)."""
    from chestnut import kernels as K
    rng = np.random.default_rng(7)
    A = (rng.standard_normal((128, 1024)) / 32).astype(np.float16)
    B = (rng.standard_normal((1024, 128)) / 32).astype(np.float16)
    C = host(K.gemm(dev(gpu, A), dev(gpu, B), b_kn=True))
    chain = OK.gemm_kchain16(A, B)
    scale = np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64))
    assert np.all(np.abs(C - chain) <= (1024 + 64 + 32) * U * scale)


@pytest.mark.parametrize('tile', [1, 2, 3, 4, 9, 15])
# N % 8 == 0 takes the LDS-staged 16-byte epilogue, N = 100 / 98 the per-element one
# (98 with split 2: the scalar split-K reduce)
@pytest.mark.parametrize('M,N,Kd,split', [(200, 136, 192, 1), (64, 64, 64, 1), (300, 520, 1024, 2), (33, 1000, 512, 4),
                                          (72, 100, 128, 1), (64, 98, 512, 2)])
def test_gemm_nt_tiles_tails(gpu, tile, M, N, Kd, split):
    from chestnut import kernels as K
    rng = np.random.default_rng(M * N + Kd + tile)
    A = rng.standard_normal((M, Kd)).astype(np.float16)
    W = rng.standard_normal((N, Kd)).astype(np.float16)
    C = host(K.gemm(dev(gpu, A), dev(gpu, W), b_kn=False, tile=tile, split_k=split))
    _gemm_check(C, A, W, transB=True)


@pytest.mark.parametrize('tile', [0, 5, 9, 15])
@pytest.mark.parametrize('N', [200, 196])
@pytest.mark.parametrize('epi', [1, 2, 3, 4])
def test_gemm_epilogues(gpu, epi, N, tile):
    from chestnut import kernels as K
    torch = gpu
    rng = np.random.default_rng(epi)
    M, Kd = 96, 256
    A = (rng.standard_normal((M, Kd)) / 8).astype(np.float16)
    W = (rng.standard_normal((N, Kd)) / 8).astype(np.float16)
    b = rng.standard_normal(N).astype(np.float32)
    acc = OK.gemm(A, W, transB=True) + b
    if epi == 4:
        C0 = rng.standard_normal((M, N)).astype(np.float32)
        out = dev(torch, C0.copy())
        K.gemm_epi(dev(torch, A), dev(torch, W), dev(torch, b), 4, out, tile=tile)
        ref = C0 + acc
        got = host(out)
        scale = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T + np.abs(b) + np.abs(C0)
        assert np.all(np.abs(got - ref) <= (Kd // 16 + 40) * U * scale)
        return
    out = torch.empty(M, N, dtype=torch.float16, device='cuda')
    K.gemm_epi(dev(torch, A), dev(torch, W), dev(torch, b), epi, out, tile=tile)
    got = host(out).astype(np.float64)
    if epi == 2:
        acc = np.maximum(acc, 0)
    if epi == 3:
        acc = OK.gelu(acc)
    ref = acc.astype(np.float32).astype(np.float16).astype(np.float64)
    # f16 rounding of an f32 value within reassociation noise: at most one f16 ulp apart
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ref) <= ulp + 1e-7)


# ------------------------------------------------------- packing / image ----
def test_pack_yuv_golden_and_full(gpu):
    from chestnut import kernels as K
    z = golden('pack_kat.npz')
    out = host(K.pack_yuv(dev(gpu, z['Y']), dev(gpu, z['U']), dev(gpu, z['V'])))
    np.testing.assert_array_equal(out, z['out'])
    rng = np.random.default_rng(3)
    Y, U_, V = (rng.integers(0, 256, (256, 512), dtype=np.uint8) for _ in range(3))
    np.testing.assert_array_equal(host(K.pack_yuv(dev(gpu, Y), dev(gpu, U_), dev(gpu, V))), OP.yuv_to_channels(Y, U_, V))


def test_frames_to_tensor_golden_and_full(gpu):
    from chestnut import kernels as K
    z = golden('i420_kat.npz')
    np.testing.assert_array_equal(host(K.frames_to_tensor(dev(gpu, z['frame']))), z['out'])
    f = np.random.default_rng(4).integers(0, 256, (384, 512), dtype=np.uint8)
    np.testing.assert_array_equal(host(K.frames_to_tensor(dev(gpu, f))), OP.frames_to_tensor(f))


def test_img_gather_sampler_kat(gpu):
    from chestnut import kernels as K
    z = golden('sampler_kat.json')
    img = np.array(z['data'], np.float32).reshape(z['height'], z['width'], z['lanes'])
    yx = np.array([[c['y'], c['x']] for c in z['cases']], np.int32)
    out = host(K.img_gather(dev(gpu, img), dev(gpu, yx)))
    np.testing.assert_array_equal(out, np.array([c['expect'] for c in z['cases']], np.float32))


@pytest.mark.parametrize('dtype,lanes', [(np.uint8, 1), (np.float16, 4), (np.float32, 4), (np.uint8, 4)])
def test_img_gather_random_oob(gpu, dtype, lanes):
    from chestnut import kernels as K
    rng = np.random.default_rng(lanes)
    A, B = 37, 53
    img = rng.integers(0, 255, (A, B, lanes)).astype(dtype)
    yx = np.stack([rng.integers(-3, A + 3, 5000), rng.integers(-3, B + 3, 5000)], 1).astype(np.int32)
    yx[:4] = [[0, 0], [A - 1, B - 1], [-1, B], [A, -1]]
    out = host(K.img_gather(dev(gpu, img), dev(gpu, yx)))
    np.testing.assert_array_equal(out.view(np.uint8), OI.gather(img, yx).view(np.uint8))


# ------------------------------------------------ attention / layernorm ----
@pytest.mark.parametrize('T,H,hd', [(512, 16, 128), (256, 8, 64), (64, 2, 64), (192, 3, 128), (384, 5, 64)])
def test_attention_vs_oracle(gpu, T, H, hd):
    from chestnut import kernels as K
    rng = np.random.default_rng(T + H)
    d = H * hd
    qkv = OM.f16r(rng.standard_normal((T, 3 * d)))
    qk = qkv[:, :2 * d].astype(np.float16)
    vt = np.ascontiguousarray(qkv[:, 2 * d:].T).astype(np.float16)
    out = host(K.attention(dev(gpu, qk), dev(gpu, vt), H, hd)).astype(np.float64)
    ref = OM.attention(qkv, H, hd)
    assert np.max(np.abs(out - ref)) <= 2.0 ** -9 * np.max(np.abs(ref))


@pytest.mark.parametrize('d,rows', [(128, 37), (512, 37), (2048, 37), (2048, 512), (1024, 1024)])
def test_layernorm_vs_oracle(gpu, d, rows):
    from chestnut import kernels as K
    rng = np.random.default_rng(d + rows)
    x = (rng.standard_normal((rows, d)) * 2 + 0.5).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    b = (0.1 * rng.standard_normal(d)).astype(np.float32)
    ref = OM.layernorm(x, g, b, 1e-5)
    y16 = host(K.layernorm(dev(gpu, x), dev(gpu, g), dev(gpu, b))).astype(np.float64)
    r16 = ref.astype(np.float32).astype(np.float16).astype(np.float64)
    assert np.all(np.abs(y16 - r16) <= np.spacing(np.abs(r16).astype(np.float16)).astype(np.float64) + 1e-7)
    y32 = host(K.layernorm(dev(gpu, x), dev(gpu, g), dev(gpu, b), out_f16=False))
    assert np.max(np.abs(y32 - ref)) <= 1e-5 * np.max(np.abs(ref))
