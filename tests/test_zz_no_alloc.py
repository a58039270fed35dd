"""GPU test of the allocation-free entry point ossm_dlinoss_forward_noalloc,
called through the C ABI and checked against ossm_dlinoss_forward (the
allocating entry point with the same kernels) to the north-star tolerance:
two calls in a row, the second smaller.

The refusal of problems above the fixed scratch's limit is checked on the
host (tests/test_library.py): a call that slipped past a regressed guard
would write look-back records beyond the array, so it is never made on a
GPU."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from tests.gpu_util import announce, assert_close, dlinoss_inputs, need_gpu, no_device_errors, to_dev, to_np

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def lib():
    need_gpu()
    from ossm_amd import _lib

    return _lib


def _call(lib, name, variant, a, g, dt, bu, out):
    L, B, P = bu.shape
    stream = torch.cuda.current_stream().cuda_stream
    return getattr(lib.load(), name)(variant, a.data_ptr(), g.data_ptr(), dt.data_ptr(), bu.data_ptr(),
                                     out.data_ptr(), L, B, P, stream)


@pytest.mark.parametrize("variant", [0, 2], ids=["imex1", "im"])
def test_noalloc_forward_matches_allocating_entry(lib, variant):
    names = {0: "imex1", 2: "im"}
    for L, B, P, seed in ((4096, 32, 128, 11), (777, 3, 70, 12)):  # config 2, then smaller
        a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=seed, variant=names[variant])
        ad, gd, dtd, bud = (to_dev(x) for x in (a, g, dt, bu))
        ref = torch.empty((L, B, P, 2), dtype=torch.complex64, device="cuda")
        got = torch.full((L, B, P, 2), float("nan"), dtype=torch.complex64, device="cuda")
        announce(f"noalloc dlinoss {names[variant]} L={L} B={B} P={P}")
        lib.check(_call(lib, "ossm_dlinoss_forward", variant, ad, gd, dtd, bud, ref))
        lib.check(_call(lib, "ossm_dlinoss_forward_noalloc", variant, ad, gd, dtd, bud, got))
        torch.cuda.synchronize()
        assert_close(to_np(got), to_np(ref), RTOL, ATOL, f"noalloc vs allocating L={L} B={B} P={P}")
        no_device_errors()



def test_noalloc_forward_under_graph_capture(lib):
    """The allocation-free forward captured into a HIP graph (after one eager
    call on the device, which looks up the fixed array's address), replayed
    five times with eager calls of the allocating entry between the replays:
    every replay matches the allocating entry to the north-star tolerance."""
    L, B, P = 2000, 8, 128
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=13, variant="imex1")
    ad, gd, dtd, bud = (to_dev(x) for x in (a, g, dt, bu))
    ref = torch.empty((L, B, P, 2), dtype=torch.complex64, device="cuda")
    got = torch.full((L, B, P, 2), float("nan"), dtype=torch.complex64, device="cuda")
    announce(f"noalloc dlinoss imex1 under graph capture L={L} B={B} P={P}")
    lib.check(_call(lib, "ossm_dlinoss_forward", 0, ad, gd, dtd, bud, ref))
    lib.check(_call(lib, "ossm_dlinoss_forward_noalloc", 0, ad, gd, dtd, bud, got))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        lib.check(_call(lib, "ossm_dlinoss_forward_noalloc", 0, ad, gd, dtd, bud, got))
    expect = to_np(ref)
    for r in range(5):
        got.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert_close(to_np(got), expect, RTOL, ATOL, f"replay {r}")
        lib.check(_call(lib, "ossm_dlinoss_forward", 0, ad, gd, dtd, bud, ref))
        torch.cuda.synchronize()
    no_device_errors()
