"""CPU oracle for the per-frame driving-model hot path.

TEST INFRASTRUCTURE ONLY.  This package is a plain numpy restatement of the
reference's algorithms for the hot path (`run_frame` and the kernels behind
it).  It may be imported only by `tests/`, by `__graft_entry__.smoke()` and by
the `cpu_baseline` leg of `bench.py`, and there only as the checker.  The
product (`chestnut-on-pc_amd/`) never imports, links or executes anything in
here, and has no CPU fallback: without the HIP library it raises.

Modules
-------
kernels  GEMV (serial-reduce analogue), GEMM (fp64 and 16-wide K-chained fp32
         emulation), RDNA4 WMMA fragment semantics, MFMA layout maps.
pack     uint8 frame packing (YUV planes -> 6 channels, NV12-style buffer ->
         6 channels) and the policy input queues.
image    image2d texel addressing with zero border (and the edge-clamp
         fallback the reference also carries).
model    the synthetic driving model's frame forward, written to round to
         f16 at exactly the points the device path stores f16.
parse    output decoding (mixture-density parse, softmax, sigmoid).

Pinning status of each function (what checks it besides its own formula) is
written in that function's docstring and checked in tests/test_oracle_*.py.
"""
