"""CPU replay of the 128x96 QKV tile's fragment epilogue (gemm.hip,
store_qkv_frag_blocks on gemm_dma_kernel with one wave column): for every
workgroup, wave and lane, the Q/K and V chunks it stores and the output
elements each chunk carries.  Every element of the QKV product must land
exactly once, at the place the attention kernel reads it from: for token t
and head dim j of head h,
  Q/K chunk (((w*H + h) * T/16 + t/16) * hd/32 + j/32) * 64 + 16*((j%32)/8) + t%16,
      element j%8 (w = 0 for Q, 1 for K);
  V chunk ((h * hd/16 + j/16) * T/32 + t/32) * 64 + 16*((t%16)/4) + j%16,
      element ((t%32)/16)*4 + t%4.
The shapes include waves whose 96 columns straddle a head, the Q/K boundary
and the K/V boundary, and a token count that leaves part of a row tile
empty.  No GPU."""
import numpy as np
import pytest

BM, BN, NWG = 128, 96, 4
WM, WN, FN = 32, 96, 3


def layout_qk(t, n, T, H, hd):
    dh = H * hd
    w, f = (1, n - dh) if n >= dh else (0, n)
    h, j = f // hd, f % hd
    return ((((w * H + h) * (T // 16) + t // 16) * (hd // 32) + j // 32) * 64 + 16 * ((j % 32) // 8) + t % 16), j % 8


def layout_v(t, n, T, H, hd):
    f = n - 2 * H * hd
    h, j = f // hd, f % hd
    return (((h * (hd // 16) + j // 16) * (T // 32) + t // 32) * 64 + 16 * ((t % 16) // 4) + j % 16,
            ((t % 32) // 16) * 4 + t % 4)


def replay(T, H, hd):
    """(buffer, chunk, element) -> (token, column) for every store of the kernel."""
    d = H * hd
    N, qk_cols, dh = 3 * d, 2 * d, d
    hs = hd.bit_length() - 1
    Mt, Nt = -(-T // BM), N // BN
    out = {}

    def put(key, val):
        assert key not in out, ('written twice', key)
        out[key] = val

    for mt in range(Mt):
        for nt in range(Nt):
            for w4 in range(NWG):
                mw, nw = mt * BM + w4 * WM, nt * BN   # wm = w4, wn = 0
                for lane in range(64):
                    r, g = lane & 15, lane >> 4
                    for j in range(FN):
                        f = nw + j * 32
                        if f >= N:
                            continue
                        if f >= qk_cols:
                            f0 = f - qk_cols
                            h, c0 = f0 >> hs, f0 & (hd - 1)
                            cbase = (h << (hs - 4)) + (c0 >> 4)
                            tpb = T >> 5
                            for blk in range(2 * (WM // 32)):
                                cb, tb = blk & 1, blk >> 1
                                if mw + tb * 32 >= T:
                                    continue
                                nl, ml = j * 32 + cb * 16 + r, tb * 32 + g * 4
                                chunk = ((cbase + cb) * tpb + (mw >> 5) + tb) * 64 + g * 16 + r
                                # lo = staged V^T row nl, tokens ml..ml+3; hi = ml+16..ml+19
                                for e in range(4):
                                    put(('v', chunk, e), (mw + ml + e, nw + nl))
                                    put(('v', chunk, 4 + e), (mw + ml + 16 + e, nw + nl))
                        else:
                            which = int(f >= dh)
                            f0 = f - which * dh
                            h, c0 = f0 >> hs, f0 & (hd - 1)
                            hbase = (which * (dh >> hs) + h) * (T >> 4)
                            kpb = hd >> 5
                            for tb in range(WM // 16):
                                if mw + tb * 16 >= T:
                                    continue
                                ml, nl = tb * 16 + r, j * 32 + g * 8
                                chunk = ((hbase + (mw >> 4) + tb) * kpb + (c0 >> 5)) * 64 + g * 16 + r
                                for e in range(8):
                                    put(('qk', chunk, e), (mw + ml, nw + nl + e))
    return out


@pytest.mark.parametrize('T,H,hd', [(512, 16, 128), (512, 8, 64), (96, 5, 64), (64, 3, 32)])
def test_qkv_tile96_epilogue_lands_every_element_once_where_attention_reads(T, H, hd):
    d = H * hd
    N, qk_cols = 3 * d, 2 * d
    assert N % BN == 0
    got = replay(T, H, hd)
    assert len(got) == T * N
    seen = set()
    for (buf, chunk, e), (t, n) in got.items():
        assert 0 <= t < T and 0 <= n < N
        if buf == 'qk':
            assert n < qk_cols and (chunk, e) == layout_qk(t, n, T, H, hd)
            assert chunk * 16 + 16 <= 2 * T * qk_cols
        else:
            assert n >= qk_cols and (chunk, e) == layout_v(t, n, T, H, hd)
            assert chunk * 16 + 16 <= 2 * T * (N - qk_cols)
        seen.add((t, n))
    assert len(seen) == T * N


def test_qkv_tile96_shapes_straddle_the_boundaries():
    # the cases above include waves across a head, the Q/K and the K/V boundary
    for T, H, hd in [(512, 16, 128), (96, 5, 64)]:
        d = H * hd
        starts = range(0, 3 * d, BN)
        assert any(s < d < s + BN for s in starts) or any(s < 2 * d < s + BN for s in starts)
        assert any((s // hd) != ((s + BN - 1) // hd) for s in starts)
