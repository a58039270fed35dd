"""GPU tests of the library's launch bookkeeping (runtime.cpp): calls from
several host threads on one stream, and refusal of HIP-graph capture.

The look-back scans draw a launch tag and a ticket base on the host, and the
backward passes leave partial sums in a per-stream workspace for the launch
that follows.  Each C call holds its (device, stream) from that bookkeeping
through its last launch, so calls from different host threads on the same
stream reach the stream whole and in the order their bookkeeping was drawn.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (announce, assert_close, dlinoss_inputs, need_gpu, no_device_errors,
                            to_dev, to_np)

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def K():
    need_gpu()
    from ossm_amd import _kernels

    return _kernels


def _selective_inputs(seed, Bz=3, D=128, L=300, N=16):
    rng = np.random.default_rng(seed)
    u = rng.normal(size=(Bz, D, L)).astype(np.float32)
    dt = np.log1p(np.exp(rng.normal(size=(Bz, D, L)) - 4.0)).astype(np.float32)
    A = np.tile(-np.arange(1, N + 1, dtype=np.float32), (D, 1))
    Bm = rng.normal(size=(Bz, L, N)).astype(np.float32)
    Cm = rng.normal(size=(Bz, L, N)).astype(np.float32)
    z = rng.normal(size=(Bz, D, L)).astype(np.float32)
    go = rng.normal(size=(Bz, D, L)).astype(np.float32)
    return u, dt, A, Bm, Cm, z, go


def test_two_host_threads_share_one_stream(K):
    """Two Python threads (ctypes releases the GIL for each call) issue D-LinOSS
    fwd+bwd and selective fwd+bwd on torch's default stream, 12 rounds each,
    at sizes inside the already-allocated scratch and workspace.  Every
    round's outputs match the oracle and no kernel raises an error bit."""
    dl = [dlinoss_inputs(700, 3, 70, seed=100 + i, variant="imex1") for i in range(2)]
    se = [_selective_inputs(200 + i) for i in range(2)]
    dl_ref = []
    for a, g, dt, bu, go in dl:
        st = oracle.dlinoss_forward("imex1", a, g, dt, bu)
        dl_ref.append((st, oracle.dlinoss_backward("imex1", a, g, dt, bu, st, go)))
    se_ref = []
    for u, dt, A, Bm, Cm, z, go in se:
        se_ref.append((oracle.selective_forward(u, dt, A, Bm, Cm, z),
                       oracle.selective_backward(go, u, dt, A, Bm, Cm, z)))
    dl_dev = [[to_dev(x) for x in case] for case in dl]
    se_dev = [[to_dev(x) for x in case] for case in se]
    announce("runtime: warm-up calls size the scratch and the workspace")
    for i in range(2):
        a, g, dt, bu, go = dl_dev[i]
        st = K.dlinoss_imex1_forward(a, g, dt, bu)
        K.dlinoss_imex1_backward(a, g, dt, bu, st, go)
        u, dts, A, Bm, Cm, z, go = se_dev[i]
        out, cs, raw = K.selective_scan_cuda(u, dts, A, Bm, Cm, z)
        K.selective_scan_cuda_backward(go, u, dts, A, Bm, Cm, z, cs, raw, 16)
    torch.cuda.synchronize()
    no_device_errors()

    rounds = 12
    results = [[] for _ in range(2)]
    errors = []
    start = threading.Barrier(2)

    def worker(i):
        try:
            start.wait()
            a, g, dt, bu, go = dl_dev[i]
            u, dts, A, Bm, Cm, z, gs = se_dev[i]
            for _ in range(rounds):
                st = K.dlinoss_imex1_forward(a, g, dt, bu)
                grads = K.dlinoss_imex1_backward(a, g, dt, bu, st, go)
                out, cs, raw = K.selective_scan_cuda(u, dts, A, Bm, Cm, z)
                sgrads = K.selective_scan_cuda_backward(gs, u, dts, A, Bm, Cm, z, cs, raw, 16)
                results[i].append((st, grads, out, sgrads))
        except Exception as exc:  # surfaced after join
            errors.append(exc)

    announce(f"runtime: two host threads x {rounds} rounds on one stream")
    threads = [threading.Thread(target=worker, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "worker threads did not finish"
    assert not errors, errors
    torch.cuda.synchronize()
    no_device_errors()
    for i in range(2):
        st_ref, (rga, rgg, rgs, rgb) = dl_ref[i]
        out_ref, sel_ref = se_ref[i]
        for st, grads, out, sgrads in results[i]:
            assert_close(to_np(st), st_ref, RTOL, ATOL, f"thread {i} states")
            assert_close(to_np(grads[3]), rgb, RTOL, ATOL, f"thread {i} grad_bu")
            for got, r, key in zip(grads[:3], (rga, rgg, rgs), ("grad_a", "grad_g", "grad_step")):
                assert_close(to_np(got), r, RTOL, 2e-5 * max(1.0, float(np.abs(r).max())),
                             f"thread {i} {key}")
            assert_close(to_np(out), out_ref, RTOL, ATOL, f"thread {i} selective out")
            for got, r, key in zip(sgrads, sel_ref, ("du", "ddt", "dA", "dB", "dC", "dz")):
                assert_close(to_np(got), r, 2e-4, 1e-4 * max(1.0, float(np.abs(r).max())),
                             f"thread {i} selective {key}")


def test_graph_capture_is_refused(K):
    """A call made while its stream is being captured into a HIP graph raises
    RuntimeError before anything is enqueued (the look-back tags and ticket
    bases are drawn on the host per call; a replay would reuse them).  Eager
    calls afterwards are unaffected."""
    a, g, dt, bu, _ = dlinoss_inputs(300, 2, 40, seed=7)
    ad, gd, dtd, bud = (to_dev(x) for x in (a, g, dt, bu))
    u, dts, A, Bm, Cm, z, _ = (to_dev(x) for x in _selective_inputs(9, Bz=2, D=64, L=100))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    announce("runtime: capture refusal")
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(RuntimeError, match="captured into a HIP graph"):
                K.dlinoss_imex1_forward(ad, gd, dtd, bud)
            with pytest.raises(RuntimeError, match="captured into a HIP graph"):
                K.selective_scan_cuda(u, dts, A, Bm, Cm, z)
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    st = K.dlinoss_imex1_forward(ad, gd, dtd, bud)
    assert_close(to_np(st), oracle.dlinoss_forward("imex1", a, g, dt, bu), RTOL, ATOL, "after capture")
    no_device_errors()
