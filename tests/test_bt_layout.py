"""CPU replay of the [K][N]-B LDS-DMA layout of gemm.hip (gemm_dma_kernel with
BT): the DMA addressing and row swizzle that fill a 64x128 stage, the per-lane
addresses of the transposed fragment reads, and the ds_read_b64_tr_b16 lane
permutation (measured on gfx950 with an in-bounds probe: within a 16-lane
group, result lane j element e = source lane 4e + j/4 element j%4) must give
every lane the MFMA 32x32x16 B operand it needs (column l%32, k 8*(l/32)..+7),
with at most two lanes' 8 bytes per LDS bank per read.  No GPU."""
import numpy as np

BN, BK, NWG, NIB = 128, 64, 4, 4


def swz(r):
    return ((r & 3) << 2) | ((r >> 3) & 1)


def fill_stage(B):
    lds = np.full(BK * BN, -1, np.int64)
    for w4 in range(NWG):
        for i in range(NIB):
            for lane in range(64):
                r = (w4 * NIB + i) * 4 + (lane >> 4)
                q = (lane & 15) ^ swz(r)
                lds[(w4 * NIB + i) * 512 + lane * 8:(w4 * NIB + i) * 512 + lane * 8 + 8] = B[r, q * 8:q * 8 + 8]
    return lds


def read_offsets(wn, j, h):
    offs = []
    for lane in range(64):
        g, a, b = lane >> 4, (lane >> 2) & 3, lane & 3
        row = 8 * (g >> 1) + 4 * h + a
        col = wn * 64 + j * 32 + 16 * (g & 1) + 4 * b
        offs.append(row * BN + (((col >> 3) ^ swz(row)) << 3) + (col & 7))
    return offs


def tr_read(lds, offs):
    src = np.array([lds[o:o + 4] for o in offs])
    out = np.empty_like(src)
    for grp in range(4):
        for jj in range(16):
            for e in range(4):
                out[16 * grp + jj, e] = src[16 * grp + 4 * e + jj // 4, jj % 4]
    return out


def test_stage_fill_is_a_swizzled_copy():
    B = np.arange(BK * BN).reshape(BK, BN)
    lds = fill_stage(B)
    assert (lds >= 0).all()
    for r in range(BK):
        for c in range(16):
            phys = c ^ swz(r)
            assert (lds[r * BN + phys * 8:r * BN + phys * 8 + 8] == B[r, c * 8:c * 8 + 8]).all()


def test_transposed_reads_give_the_mfma_b_operand():
    rng = np.random.default_rng(0)
    B = rng.integers(0, 1 << 30, (BK, BN))
    lds = fill_stage(B)
    for wn in range(2):
        for j in range(2):
            for kk in range(4):
                frag = np.concatenate([tr_read(lds, [kk * 16 * BN + o for o in read_offsets(wn, j, h)])
                                       for h in range(2)], axis=1)
                for lane in range(64):
                    k = kk * 16 + 8 * (lane // 32) + np.arange(8)
                    assert (frag[lane] == B[k, wn * 64 + j * 32 + lane % 32]).all()


def test_transposed_reads_use_each_bank_at_most_twice():
    for wn in range(2):
        for j in range(2):
            for h in range(2):
                hits = {}
                for o in read_offsets(wn, j, h):
                    for bank in ((o * 2 // 4) % 64, (o * 2 // 4 + 1) % 64):   # 8 bytes = 2 banks
                        hits[bank] = hits.get(bank, 0) + 1
                assert max(hits.values()) <= 2 and len(hits) == 64


def test_register_staged_b_layout_and_banks():
    """gemm_kn_rb_kernel: group thread tg (lane l of wave w, tg = 64w + l) holds
    rows 2kp, 2kp+1 (kp = tg >> 3) of columns 8no .. 8no+7 (no = tg & 7) of
    the step's 64 x 64 [K][N] B tile; its write j puts column n = 8no + (j ^ x)
    (x = l >> 5) as the dword (B[k][n], B[k+1][n]), k = 2kp, at halves offset
    n*64 + ((k>>3) ^ f(n))*8 + (k&7), f(n) = ((n>>1) ^ (n>>4)) & 7.  The 256
    threads x 8 writes must fill every half of the stage once, as the [N][K]
    layout the 16-byte fragment reads address (row n, physical chunk =
    chunk ^ f(n)); every write instruction's 64 lanes must hit 64 distinct
    banks, and every fragment read's 16-lane pass (rows base + l%32, chunk
    2kk + l/32) 64 distinct banks."""
    f = lambda n: ((n >> 1) ^ (n >> 4)) & 7                     # noqa: E731
    bank = lambda h: (h * 2 // 4) % 64                           # noqa: E731
    rng = np.random.default_rng(3)
    B = rng.integers(0, 1 << 30, (64, 64))
    lds = np.full(64 * 64, -1, np.int64)
    for w in range(4):
        for j in range(8):
            banks = set()
            for lane in range(64):
                tg = 64 * w + lane
                kp, no, x = tg >> 3, tg & 7, lane >> 5
                n, k = 8 * no + (j ^ x), 2 * kp
                off = n * 64 + (((k >> 3) ^ f(n)) << 3) + (k & 7)
                assert lds[off] == -1 and lds[off + 1] == -1
                lds[off], lds[off + 1] = B[k, n], B[k + 1, n]
                banks.add(bank(off))
            assert len(banks) == 64
    assert (lds >= 0).all()
    for n in range(64):
        for k in range(64):
            assert lds[n * 64 + (((k >> 3) ^ f(n)) << 3) + (k & 7)] == B[k, n]
    for base in (0, 32):
        for kk in range(4):
            for p in range(4):
                banks = []
                for lane in range(16 * p, 16 * p + 16):
                    n, c = base + (lane & 31), 2 * kk + (lane >> 5)
                    o = n * 64 + ((c ^ f(n)) << 3)
                    banks += [(bank(o) + d) % 64 for d in range(4)]
                assert sorted(banks) == list(range(64))
