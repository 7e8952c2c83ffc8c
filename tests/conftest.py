import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, 'chestnut-on-pc_amd')
GOLDEN = os.path.join(ROOT, 'tests', 'golden')
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs an MI355X (gfx950) GPU and the built libchestnut.so')


def golden(name):
    path = os.path.join(GOLDEN, name)
    if name.endswith('.npz'):
        return np.load(path, allow_pickle=False)
    import json
    with open(path) as fh:
        return json.load(fh)


@pytest.fixture(scope='session')
def gpu():
    """torch with a visible GPU and the native library loaded; fails (never
    silently falls back) when either is missing on a GPU run."""
    import torch
    assert torch.cuda.is_available(), 'GPU test run without a visible GPU'
    from chestnut import _lib
    _lib.lib()
    print(f'[gpu] device={torch.cuda.get_device_name(0)} lib={_lib.LIB_PATH}', flush=True)
    return torch
