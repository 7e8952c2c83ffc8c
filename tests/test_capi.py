"""The C-ABI library loads, exports every symbol include/chestnut.h declares,
and its host-side validation and error convention work (no GPU needed:
nothing here launches a kernel)."""
import ctypes

import numpy as np
import pytest

from chestnut import _lib
from chestnut import spec as S


def test_header_symbols_exported():
    L = _lib.lib()
    names = _lib.header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # and the Python binding declares a signature for every one of them
    assert set(names) == set(_lib._SIGS), set(names) ^ set(_lib._SIGS)


def test_version_and_last_error():
    L = _lib.lib()
    a, b = ctypes.c_int(), ctypes.c_int()
    assert L.ck_version(ctypes.byref(a), ctypes.byref(b)) == 0
    assert (a.value, b.value) == (0, 1)


def test_bad_spec_raises_with_message():
    with pytest.raises(RuntimeError, match='spec json'):
        _lib.call('ck_create', b'{"d_model": 12', ctypes.byref(ctypes.c_void_p()))
    with pytest.raises(RuntimeError, match='missing key'):
        _lib.call('ck_create', b'{"stem": [8]}', ctypes.byref(ctypes.c_void_p()))
    bad = dict(S.get_spec('tiny'), n_heads=3)
    with pytest.raises(RuntimeError, match='n_heads'):
        _lib.call('ck_create', S.spec_json(bad).encode(), ctypes.byref(ctypes.c_void_p()))
    odd = dict(S.get_spec('tiny'), camera=dict(S.ROAD_CAMERA, width=1927))
    with pytest.raises(RuntimeError, match='camera needs an even width'):
        _lib.call('ck_create', S.spec_json(odd).encode(), ctypes.byref(ctypes.c_void_p()))


@pytest.mark.parametrize('change,message', [
    (dict(stem=[8, 16, 'x', 64, 64]), 'stem width must be a number'),
    (dict(stem=[8, 16, 32, 64, 0]), 'stem widths must be positive'),
    (dict(n_layers=0), 'must be positive'),
    (dict(img_h=0), 'must be positive'),
    (dict(feat_hist=-3), 'must be positive'),
    (dict(d_model=256, n_heads=8, head_dim=32), 'head_dim must be 64 or 128'),
    (dict(feat_len=20, hidden=20), 'feat_len must be a multiple of 8'),
    (dict(d_ff=512.5), 'd_ff must be an integer'),
    (dict(frame_skip=1e12), 'frame_skip must be an integer'),
    (dict(ln_eps=0), 'ln_eps must be a positive number'),
    (dict(outputs=[['plan', 0]]), 'output sizes must be positive'),
    (dict(outputs=[[3, 10]]), 'outputs entries are'),
    (dict(gemm_config={'blk0.up': ['a', 1]}), 'gemm_config tile must be a number'),
])
def test_spec_fields_are_checked_before_any_allocation(change, message):
    # parse_spec runs before the engine touches the GPU, so a bad field is
    # reported by name here, not as a HIP failure
    bad = dict(S.get_spec('tiny'), **change)
    with pytest.raises(RuntimeError, match=message):
        _lib.call('ck_create', S.spec_json(bad).encode(), ctypes.byref(ctypes.c_void_p()))


def test_nv12_bytes():
    # Y plane 2048 x 1216 plus 604 UV rows of 2048 bytes
    assert S.nv12_bytes(S.ROAD_CAMERA) == 2048 * 1216 + 604 * 2048


def test_kernel_entry_validation_rejects_before_launch():
    with pytest.raises(RuntimeError, match='K must be a multiple of 8'):
        _lib.call('ck_gemv', ctypes.c_void_p(16), ctypes.c_void_p(16), None, ctypes.c_void_p(16), 4, 12, 16, 0, 0,
                  None)
    with pytest.raises(RuntimeError, match='16-byte aligned'):
        _lib.call('ck_gemv', ctypes.c_void_p(18), ctypes.c_void_p(16), None, ctypes.c_void_p(16), 4, 16, 16, 0, 0,
                  None)
    with pytest.raises(RuntimeError, match='null'):
        _lib.call('ck_img_gather', None, 1, 2, 4, 4, None, 1, None, None)
    with pytest.raises(RuntimeError, match='T must be'):
        _lib.call('ck_attention', ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 100, 2, 64, None)
    with pytest.raises(RuntimeError, match='d must be one of'):
        _lib.call('ck_layernorm', ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16),
                  ctypes.c_void_p(16), 1, 4, 100, 1e-5, None)


def test_gemm_planner_host_logic():
    t, s, nb = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_size_t()
    # config 1: 1024 x 1024 output, K = 6144, [K][N] B -> 128 tiles of 128x64 (B through
    # registers), split 2 to fill 256 CUs; workspace: the 2 partial planes, no transposed B
    _lib.call('ck_gemm_workspace', 1024, 1024, 6144, 1, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    assert t.value == 2 and s.value == 2 and nb.value == 2 * 1024 * 1024 * 4
    # the same with B as [N][K]: 64 tiles of 128x128, split 4
    t, s = ctypes.c_int(0), ctypes.c_int(0)
    _lib.call('ck_gemm_workspace', 1024, 1024, 6144, 0, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    assert t.value == 1 and s.value == 4 and nb.value == 4 * 1024 * 1024 * 4
    # tile 1 reads the [K][N] B transposed out of LDS: the partial planes only
    t, s = ctypes.c_int(1), ctypes.c_int(4)
    _lib.call('ck_gemm_workspace', 1024, 1024, 6144, 1, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    assert nb.value == 4 * 1024 * 1024 * 4
    # one K-group (tile 5) transposes B into the workspace tail first
    t, s = ctypes.c_int(5), ctypes.c_int(4)
    _lib.call('ck_gemm_workspace', 1024, 1024, 6144, 1, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    assert nb.value == 4 * 1024 * 1024 * 4 + 1024 * 6144 * 2
    t, s = ctypes.c_int(0), ctypes.c_int(0)
    # 1B MLP-up: 512 x 8192 -> 256 tiles, no split
    _lib.call('ck_gemm_workspace', 512, 8192, 2048, 0, ctypes.byref(t), ctypes.byref(s), ctypes.byref(nb))
    assert t.value == 1 and s.value == 1 and nb.value == 0
    with pytest.raises(RuntimeError, match='multiple of 64'):
        _lib.call('ck_gemm_workspace', 64, 64, 100, 0, ctypes.byref(ctypes.c_int(0)), ctypes.byref(ctypes.c_int(0)),
                  ctypes.byref(nb))


def test_output_slices_match_python_spec():
    sl = S.output_slices('big_driving_1b')
    assert list(sl) == ['plan', 'lead', 'lead_prob', 'lane_lines', 'lane_lines_prob', 'hidden_state']
    assert sl['hidden_state'].stop == S.output_size('big_driving_1b')


def test_engine_requires_library_no_fallback(monkeypatch, tmp_path):
    """Without the built library the product raises; there is no CPU path."""
    monkeypatch.setattr(_lib, '_lib', None)
    monkeypatch.setattr(_lib, 'LIB_PATH', str(tmp_path / 'missing.so'))
    from chestnut import Engine
    with pytest.raises(RuntimeError, match='not built'):
        Engine('tiny')


def test_operand_stream_rejects_bad_arguments():
    """Argument checks run before any device call (so on the CPU too)."""
    import ctypes
    from chestnut._lib import call
    v = ctypes.c_float()
    for args, msg in (((256, 512, 320, 4, 1, 1), 'mode 0-3'), ((200, 512, 320, 0, 1, 1), 'multiple of 128'),
                      ((256, 512, 100, 0, 1, 1), 'K of 64'), ((256, 512, 320, 0, 0, 1), 'copies'),
                      ((256, 512, 320, 3, 1, 1), 'tile width')):
        with pytest.raises(RuntimeError, match=msg):
            call('ck_time_operand_stream', *args, ctypes.byref(v), None)
