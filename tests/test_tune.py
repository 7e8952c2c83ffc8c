"""Candidate generation and config expansion of chestnut.tune (host logic)."""
from chestnut import spec as S
from chestnut import tune as TU


def test_candidates_respect_epilogue_and_grid():
    sh = TU.shapes(S.get_spec('big_driving_1b'))
    M, N, K, kind, _ = sh['qkv']
    c = TU.candidates(M, N, K, kind)
    assert (5, 1) in c and (1, 1) in c and (10, 1) in c                   # 10: the 128x96 QKV tile
    assert all(s == 1 for _, s in c) and all(t != 9 for t, _ in c)       # fragment epilogue: split 1, no 256-row tile
    M, N, K, kind, _ = sh['o']
    c = TU.candidates(M, N, K, kind)
    assert (2, 2) in c and (1, 4) in c and (4, 1) in c
    assert all(s <= 8 for _, s in c)                                       # the LayerNorm sums <= 8 partials
    for t, s in c:
        bm, bn = TU.TILES[t]
        grid = -(-M // bm) * -(-N // bn) * s
        assert 64 <= grid <= 1024 and K % (64 * s) == 0
    assert all(t != 10 for t, _ in c)                                      # 128x96 serves the QKV epilogue only
    M, N, K, kind, _ = sh['up']
    assert all(s == 1 for _, s in TU.candidates(M, N, K, kind))            # GELU epilogue is not split


def test_config_for_every_layer():
    sp = S.get_spec('driving_39m')
    cfg = TU.config_for(sp, {'o': (2, 2), 'down': (5, 4)})
    assert len(cfg) == 2 * sp['n_layers']
    assert cfg['blk0.o'] == [2, 2] and cfg[f'blk{sp["n_layers"] - 1}.down'] == [5, 4]


def test_stem_and_embed_shapes():
    sp = S.get_spec('big_driving_1b')
    sh = TU.shapes(sp)
    assert sh['stem0'] == (64 * 128, 32, 128, 'reduce', 2)          # 9 x 12 channels padded to 128
    assert sh['stem4'] == (4 * 8, 512, 9 * 256, 'conv', 2)          # implicit conv: no tile 9
    assert sh['embed'] == (512, 2048, 64, 'reduce', 1)
    assert TU.entry_names(sp, 'stem3') == ['stem3.conv'] and TU.entry_names(sp, 'embed') == ['embed']
    M, N, K, kind, b = sh['stem4']
    c = TU.candidates(M, N, K, kind, b)
    assert c and all(K % (64 * s) == 0 for _, s in c)
    assert all(t <= 8 or t == 15 for t, _ in c) and any(t == 15 for t, _ in c)   # implicit conv: LDS-DMA tiles 1-8, 15
    assert any(s > 1 for _, s in c)
