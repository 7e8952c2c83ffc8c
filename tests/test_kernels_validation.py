"""The torch harness (chestnut.kernels) rejects mismatched tensors with
ValueError before anything reaches the native library: wrong dtype, a shape
that disagrees with the sizes derived from the other operands, a
non-contiguous view, a tensor that is not on the current CUDA device.
Shape checks run before the device check, so on the CPU every argument's
check is reachable with CPU tensors."""
import pytest
import torch

from chestnut import kernels as K

f16, f32, i16, u8, i32 = torch.float16, torch.float32, torch.int16, torch.uint8, torch.int32


def z(*shape, dtype=f32):
    return torch.zeros(*shape, dtype=dtype)


CASES = [
    # gemv: W [rows, K], x [K], bias [rows], out [rows]
    ('gemv x length', lambda: K.gemv(z(8, 64, dtype=f16), z(60)), "x must have shape \\(64,\\)"),
    ('gemv bias length', lambda: K.gemv(z(8, 64, dtype=f16), z(64), bias=z(9)), "bias must have shape \\(8,\\)"),
    ('gemv out length', lambda: K.gemv(z(8, 64, dtype=f16), z(64), out=z(7)), "out must have shape \\(8,\\)"),
    ('gemv x dtype', lambda: K.gemv(z(8, 64, dtype=f16), z(64, dtype=f16)), 'x must be torch.float32'),
    ('gemv act', lambda: K.gemv(z(8, 64, dtype=f16), z(64), act=2), 'act must be'),
    # gemm: A [M, K], B [K, N] or [N, K], bias [N], out [M, N]
    ('gemm B K mismatch (KN)', lambda: K.gemm(z(16, 64, dtype=f16), z(128, 32, dtype=f16)), 'B must have shape'),
    ('gemm B K mismatch (NK)', lambda: K.gemm(z(16, 64, dtype=f16), z(32, 128, dtype=f16), b_kn=False),
     'B must have shape'),
    ('gemm out shape', lambda: K.gemm(z(16, 64, dtype=f16), z(64, 32, dtype=f16), out=z(16, 33)),
     'out must have shape'),
    ('gemm out dtype', lambda: K.gemm(z(16, 64, dtype=f16), z(64, 32, dtype=f16), out=z(16, 32, dtype=f16)),
     'out must be torch.float32'),
    ('gemm bias length', lambda: K.gemm(z(16, 64, dtype=f16), z(64, 32, dtype=f16), bias=z(16)),
     "bias must have shape \\(32,\\)"),
    ('gemm non-contiguous A', lambda: K.gemm(z(64, 16, dtype=f16).t(), z(64, 32, dtype=f16)), 'A must be contiguous'),
    # gemm_epi: out f16 for epi 1-3, f32 for epi 4, [M, N]
    ('gemm_epi out dtype f16', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(32), 3, z(16, 32)),
     'out must be torch.float16'),
    ('gemm_epi out dtype f32', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(32), 4,
                                                  z(16, 32, dtype=f16)), 'out must be torch.float32'),
    ('gemm_epi out shape', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(32), 1,
                                              z(32, 16, dtype=f16)), 'out must have shape'),
    ('gemm_epi W K', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 32, dtype=f16), z(32), 1, z(16, 32, dtype=f16)),
     'W must have shape'),
    ('gemm_epi bias', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(31), 1, z(16, 32, dtype=f16)),
     'bias must have shape'),
    ('gemm_epi epi', lambda: K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(32), 5, z(16, 32)),
     'epi must be'),
    # the rest
    ('wmma fragC shape', lambda: K.wmma_rdna4(z(2, 32, 8, dtype=i16), z(2, 32, 8, dtype=i16), z(1, 32, 8)),
     'fragC must have shape'),
    ('mfma B shape', lambda: K.mfma_kat(0, z(16, 32, dtype=i16), z(16, 32, dtype=i16)), 'B must have shape'),
    ('pack_yuv U shape', lambda: K.pack_yuv(z(8, 8, dtype=u8), z(8, 6, dtype=u8), z(8, 8, dtype=u8)),
     'U must have shape'),
    ('frames_to_tensor rows', lambda: K.frames_to_tensor(z(10, 8, dtype=u8)), 'frame must be'),
    ('img_gather yx', lambda: K.img_gather(z(4, 4, 4), z(5, 3, dtype=i32)), 'yx must have shape'),
    ('attention vt', lambda: K.attention(z(64, 256, dtype=f16), z(64, 128, dtype=f16), 2, 64), 'vt must have shape'),
    ('attention qk', lambda: K.attention(z(64, 200, dtype=f16), z(128, 64, dtype=f16), 2, 64), 'qk must have shape'),
    ('layernorm g', lambda: K.layernorm(z(4, 128), z(64), z(128)), 'g must have shape'),
    ('warp short frame', lambda: K.warp_nv12(z(1000, dtype=u8), z(1000, dtype=u8), z(3, 3), z(3, 3), 1928, 1208,
                                             2048, 1216), 'must hold'),
    ('warp out shape', lambda: K.warp_nv12(z(2048 * 1216 + 604 * 2048, dtype=u8), z(2048 * 1216 + 604 * 2048, dtype=u8),
                                           z(3, 3), z(3, 3), 1928, 1208, 2048, 1216, out=z(2, 6, 64, 256, dtype=u8)),
     'out must have shape'),
]


@pytest.mark.parametrize('name,fn,msg', CASES, ids=[c[0] for c in CASES])
def test_mismatch_raises_value_error(name, fn, msg):
    with pytest.raises(ValueError, match=msg):
        fn()


def test_well_formed_cpu_tensors_stop_at_the_device_check():
    """Every shape agrees: the only objection left is that the tensors are not
    on a CUDA device (nothing reaches the library)."""
    with pytest.raises(ValueError, match='must be a CUDA tensor'):
        K.gemm(z(16, 64, dtype=f16), z(64, 32, dtype=f16), bias=z(32), out=z(16, 32))
    with pytest.raises(ValueError, match='must be a CUDA tensor'):
        K.gemv(z(8, 64, dtype=f16), z(64), bias=z(8), out=z(8))
    with pytest.raises(ValueError, match='must be a CUDA tensor'):
        K.gemm_epi(z(16, 64, dtype=f16), z(32, 64, dtype=f16), z(32), 3, z(16, 32, dtype=f16))
