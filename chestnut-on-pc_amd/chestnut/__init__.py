"""chestnut: MI355X (gfx950) per-frame driving-model hot path.

    from chestnut import Engine, load
    ns = load('big_driving_1b')            # run_frame, out_slices, img, make_warped, PACKED
    out = ns.run_frame(ns.make_warped(128), ns.PACKED)

Submodules: engine (frame engine), kernels (per-kernel entry points on torch
tensors), spec (model specs and seeded weights), parse (output decode),
_lib (ctypes binding of include/chestnut.h).
"""
from .engine import Engine, load  # noqa: F401
from . import spec  # noqa: F401
