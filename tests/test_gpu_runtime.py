"""GPU tests of the library's launch bookkeeping (runtime.cpp): calls from
several host threads on one stream, HIP-graph capture and replay, and the
failure path of the look-back protocol.

The look-back scans draw each workgroup's order and the launch's record tag
from a per-stream ticket counter on the device (grids of at most a quarter
as many workgroups as CUs, outside capture, take the workgroup index and a
host-chosen tag instead), and some backward passes leave partial sums in a per-stream
workspace for the launch that follows.  Each C
call holds its (device, stream) through its last launch, so calls from
different host threads on the same stream reach the stream whole, and a
captured call draws fresh orders and tags on every replay.
"""

from __future__ import annotations

import threading
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (announce, assert_close, assert_parity, dlinoss_inputs, need_gpu,
                            no_device_errors, to_dev, to_np)

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


def _dl_call(K, args, go):
    st = K.dlinoss_imex1_forward(*args)
    return [st] + list(K.dlinoss_imex1_backward(*args, st, go))


def _errors_on(stream) -> int:
    from ossm_amd import _lib

    with torch.cuda.stream(stream):
        return _lib.device_error_bits()


def test_graph_capture_replays_dlinoss_config2(K):
    """D-LinOSS imex1 forward + backward at config 2 (B=32, L=4096, P=128)
    captured into a HIP graph after an eager warm-up on the capture stream,
    replayed 10 times with eager calls on the same stream and host
    synchronisations between the replays: every replay's states and gradients
    equal the eager result (rtol 1e-4; the look-back may associate carries
    differently per run), and no protocol error is raised."""
    L, B, P = 4096, 32, 128
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=21, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    god = to_dev(go)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce("runtime: graph capture dlinoss config 2")
    with torch.cuda.stream(side):
        eager = [to_np(x) for x in _dl_call(K, args, god)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = _dl_call(K, args, god)
    names = ("states", "grad_a", "grad_g", "grad_step", "grad_bu")
    small = [x[:300].contiguous() for x in (args[3],)]
    for r in range(10):
        graph.replay()
        torch.cuda.synchronize()
        for got, ref, name in zip(outs, eager, names):
            atol = ATOL if name in ("states", "grad_bu") else 2e-5 * max(1.0, float(np.abs(ref).max()))
            assert_close(to_np(got), ref, RTOL, atol, f"replay {r} {name}")
        with torch.cuda.stream(side):  # eager work on the capture stream between replays
            K.dlinoss_imex1_forward(*args[:3], small[0])
        side.synchronize()
    assert _errors_on(side) == 0


def test_graph_capture_replays_selective(K):
    """The selective scan forward + backward (gated) captured after an eager
    warm-up and replayed 5 times: every replay equals the eager result
    bitwise (the selective scan is deterministic)."""
    u, dt, A, Bm, Cm, z, go = (to_dev(x) for x in _selective_inputs(31, Bz=8, D=128, L=400))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    announce("runtime: graph capture selective")

    def step():
        out, ck, raw = K.selective_scan_cuda(u, dt, A, Bm, Cm, z)
        return [out] + list(K.selective_scan_cuda_backward(go, u, dt, A, Bm, Cm, z, ck, raw, 16))

    with torch.cuda.stream(side):
        eager = [to_np(x) for x in step()]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        outs = step()
    for r in range(5):
        graph.replay()
        torch.cuda.synchronize()
        for got, ref, name in zip(outs, eager, ("out", "du", "ddt", "dA", "dB", "dC", "dz")):
            assert np.array_equal(to_np(got), ref), f"replay {r} {name}"
    assert _errors_on(side) == 0


def test_graph_capture_refused_when_scratch_would_grow(K):
    """On a stream with no look-back scratch yet (no eager call), a captured
    call would have to allocate: it raises RuntimeError before anything is
    enqueued, and eager calls afterwards are unaffected."""
    a, g, dt, bu, _ = dlinoss_inputs(300, 2, 40, seed=7)
    ad, gd, dtd, bud = (to_dev(x) for x in (a, g, dt, bu))
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    announce("runtime: capture refusal")
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(RuntimeError, match="would have to grow"):
                K.dlinoss_imex1_forward(ad, gd, dtd, bud)
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    st = K.dlinoss_imex1_forward(ad, gd, dtd, bud)
    assert_close(to_np(st), oracle.dlinoss_forward("imex1", a, g, dt, bu), RTOL, ATOL, "after capture")
    no_device_errors()


def test_protocol_failure_gives_nan_not_garbage(K, monkeypatch):
    """With the stream's ticket counter knocked out of step from the host (as
    a launch that did not run to its end would leave it), every workgroup of
    the next look-back launch draws an out-of-range ticket: the launch raises
    the bad-ticket bit, the chunks that needed a carry come out NaN (the first
    chunk, which needs none, is still right), and after the error check the
    next call is correct again.  Forward and backward of D-LinOSS, and the
    LRU and selective D-LinOSS forwards.  These grids are small enough for
    dispatch order, which draws no ticket, so ticket order is forced."""
    from ossm_amd import _lib

    monkeypatch.setenv("OSSM_SCAN_ORDER", "ticket")
    monkeypatch.setattr(_lib, "CHECK_DEVICE_ERRORS", False)  # the bits are read here

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    L, B, P = 1000, 2, 64
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=41, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    ref = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    rgrads = oracle.dlinoss_backward("imex1", a, g, dt, bu, ref, go)
    announce("runtime: protocol failure -> NaN")
    K.dlinoss_imex1_forward(*args)  # the stream's scratch exists
    assert _lib.device_error_bits() == 0
    skew = 1 << 20  # far above any launch's workgroup count, far below 2^32

    _lib.check(lib.ossm_test_skew_tickets(stream, skew))
    st = to_np(K.dlinoss_imex1_forward(*args))
    assert _lib.device_error_bits() == 2  # bad ticket; the check realigns the counter
    assert np.isfinite(st[:128]).all()  # the first chunk (128 or 256 steps) needs no carry
    assert_close(st[:128], ref[:128], RTOL, ATOL, "first chunk")
    assert np.isnan(st[256:]).all()

    st = K.dlinoss_imex1_forward(*args)
    _lib.check(lib.ossm_test_skew_tickets(stream, skew))
    grads = [to_np(x) for x in K.dlinoss_imex1_backward(*args, st, to_dev(go))]
    assert _lib.device_error_bits() == 2
    assert all(np.isnan(x).all() for x in grads[:3])  # sums over every chunk
    # reverse scan: the last chunk (128 steps here) needs no carry
    assert np.isnan(grads[3][:L - 256]).all() and np.isfinite(grads[3][L - 100:]).all()

    # LRU forward (diagonal scan) and selective D-LinOSS forward
    lam = torch.polar(torch.rand(P, device="cuda") * 0.5 + 0.5, torch.rand(P, device="cuda"))
    bseq = torch.randn(L, B, P, 2, device="cuda")
    K.lru_scan(lam.real.contiguous(), lam.imag.contiguous(), bseq)
    _lib.check(lib.ossm_test_skew_tickets(stream, skew))
    y = to_np(K.lru_scan(lam.real.contiguous(), lam.imag.contiguous(), bseq))
    assert _lib.device_error_bits() == 2
    assert np.isnan(y[L - 100:]).all() and np.isfinite(y[:64]).all()  # last chunk / first
    A = to_dev(a)[None, None].expand(L, B, P).contiguous()
    sdl = lambda: K.sdlinoss_imex1_forward(A, A * 0 + to_dev(g), A * 0 + to_dev(dt), args[3])  # noqa: E731
    sdl()
    _lib.check(lib.ossm_test_skew_tickets(stream, skew))
    y = to_np(sdl())
    assert _lib.device_error_bits() == 2
    assert np.isnan(y[L - 100:]).all() and np.isfinite(y[:64]).all()  # last chunk / first

    # back in step: correct and error-free
    st = to_np(K.dlinoss_imex1_forward(*args))
    assert_close(st, ref, RTOL, ATOL, "after recovery")
    grads = K.dlinoss_imex1_backward(*args, to_dev(st), to_dev(go))
    assert_close(to_np(grads[3]), rgrads[3], RTOL, ATOL, "grad_bu after recovery")
    no_device_errors()


# grids of 528 and 1,088 chunks (16 x 16 tiles): more than the device holds at once,
# so the forward runs persistent (each workgroup two to five chunks, ragged counts)
@pytest.mark.parametrize("shape", [(8292, 8, 128), (4200, 32, 128)], ids=lambda s: "x".join(map(str, s)))
def test_persistent_forward_matches_oracle_and_one_chunk_per_workgroup(K, monkeypatch, shape):
    """The persistent D-LinOSS forward (ticket order, fewer workgroups than
    chunks, each drawing its next ticket while it stores) against the oracle
    and against the one-workgroup-per-chunk launch (OSSM_OSC_PERSIST=0), twice
    in a row on one stream; the selective D-LinOSS forward with parameters
    constant over time (the same kernel, another model) likewise."""
    L, B, P = shape
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=61, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    ref = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    st64 = oracle.dlinoss_forward("imex1", *(x.astype(np.float64) for x in (a, g, dt)),
                                  bu.astype(np.complex128))
    announce(f"runtime: persistent forward L={L} B={B} P={P}")
    for mode in ("1", "0", "1"):
        monkeypatch.setenv("OSSM_OSC_PERSIST", mode)
        st = to_np(K.dlinoss_imex1_forward(*args))
        assert_parity(st, ref, st64, RTOL, ATOL, f"persist={mode} states")
    from tests.test_gpu_sdlinoss import sdl_inputs

    A, G, S, sbu, _ = sdl_inputs("imex1", "m", L, B, P, seed=62)
    sref = oracle.sdlinoss_forward("imex1", A, G, S, sbu)
    s64 = oracle.sdlinoss_forward("imex1", *(x.astype(np.float64) for x in (A, G, S)),
                                  sbu.astype(np.complex128))
    for mode in ("1", "0"):
        monkeypatch.setenv("OSSM_OSC_PERSIST", mode)
        out = to_np(K.sdlinoss_imex1_forward(to_dev(A), to_dev(G), to_dev(S), to_dev(sbu)))
        assert_parity(out, sref, s64, RTOL, ATOL, f"sdlinoss persist={mode}")
    no_device_errors()


def test_protocol_failure_persistent_forward(K, monkeypatch):
    """The failure path of the persistent forward: with the ticket counter out
    of step every draw is out of range, every chunk is still taken exactly
    once (orders modulo the chunk count), the chunks that needed a carry are
    NaN, the first chunk is right, and the next call is correct."""
    from ossm_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    L, B, P = 8292, 8, 128  # 528 chunks of 256 steps: persistent
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=63, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    ref = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    announce("runtime: persistent forward protocol failure -> NaN")
    monkeypatch.setenv("OSSM_SCAN_ORDER", "ticket")
    monkeypatch.setattr(_lib, "CHECK_DEVICE_ERRORS", False)  # the bits are read here
    K.dlinoss_imex1_forward(*args)
    assert _lib.device_error_bits() == 0
    _lib.check(lib.ossm_test_skew_tickets(stream, 1 << 20))
    st = to_np(K.dlinoss_imex1_forward(*args))
    assert _lib.device_error_bits() == 2
    assert_close(st[:256], ref[:256], RTOL, ATOL, "first chunk")
    assert np.isnan(st[256:]).all()
    st = to_np(K.dlinoss_imex1_forward(*args))
    st64 = oracle.dlinoss_forward("imex1", *(x.astype(np.float64) for x in (a, g, dt)),
                                  bu.astype(np.complex128))
    assert_parity(st, ref, st64, RTOL, ATOL, "after recovery")  # L = 8292: fp64 arbiter
    no_device_errors()


def test_protocol_failure_raises_with_device_error_checks(K, monkeypatch):
    """With OSSM_CHECK_DEVICE_ERRORS=1 (here set on the module), a call whose
    kernels raise a protocol error bit raises RuntimeError naming the bits, and
    the calls after it are correct and raise nothing."""
    from ossm_amd import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    L, B, P = 1000, 2, 64
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=64, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    announce("runtime: protocol failure raises under device error checks")
    monkeypatch.setenv("OSSM_SCAN_ORDER", "ticket")
    monkeypatch.setattr(_lib, "CHECK_DEVICE_ERRORS", True)
    K.dlinoss_imex1_forward(*args)
    # not through _lib.check: its device check would put the counter back in step
    assert lib.ossm_test_skew_tickets(stream, 1 << 20) == 0
    with pytest.raises(RuntimeError, match="device error bits 0x2"):
        K.dlinoss_imex1_forward(*args)
    st = to_np(K.dlinoss_imex1_forward(*args))
    assert_close(st, oracle.dlinoss_forward("imex1", a, g, dt, bu), RTOL, ATOL, "after the error")


def _dl_truth(a, g, dt, bu, go):
    """fp32 oracle states and gradients, and the fp64 ones as arbiter."""
    st = oracle.dlinoss_forward("imex1", a, g, dt, bu)
    grads = oracle.dlinoss_backward("imex1", a, g, dt, bu, st, go)
    a64, g64, d64 = (x.astype(np.float64) for x in (a, g, dt))
    b64, go64 = bu.astype(np.complex128), go.astype(np.complex128)
    st64 = oracle.dlinoss_forward("imex1", a64, g64, d64, b64)
    return st, grads, st64, oracle.dlinoss_backward("imex1", a64, g64, d64, b64, st64, go64)


# forward grids of 16, 64 and 256 workgroups: the device has 256 CUs, so the
# default (auto) takes dispatch order for the first two and ticket order for
# the third
@pytest.mark.parametrize("shape", [(1000, 2, 64), (1024, 8, 64), (4096, 8, 128)],
                         ids=lambda s: "x".join(map(str, s)))
def test_scan_orders_alternate_on_one_stream(K, monkeypatch, shape):
    """D-LinOSS imex1 forward + backward and the LRU forward, launched in
    ticket, dispatch and automatic order (OSSM_SCAN_ORDER, read per call) in
    turn on one stream, each call on the other of two input sets: every result
    matches the oracle.  A launch that took a look-back record, or the
    zero-filled flag of the parameter gradients, left by the previous launch
    (of the other order, on other inputs) would carry that launch's values:
    the tags the host chooses for dispatch order and those drawn on the device
    for ticket order are disjoint."""
    L, B, P = shape
    sets = []
    for seed in (51, 52):
        a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=seed, variant="imex1")
        lam = (np.random.default_rng(seed).uniform(0.5, 1.0, P)
               * np.exp(1j * np.random.default_rng(seed + 9).uniform(0, 3, P))).astype(np.complex64)
        sets.append(dict(dev=[to_dev(x) for x in (a, g, dt, bu)], go=to_dev(go),
                         truth=_dl_truth(a, g, dt, bu, go),
                         lam=(torch.from_numpy(lam.real.copy()).cuda(), torch.from_numpy(lam.imag.copy()).cuda()),
                         lru=(oracle.diag_forward(lam, bu),
                              oracle.diag_forward(lam.astype(np.complex128), bu.astype(np.complex128)))))
    names = ("grad_a", "grad_g", "grad_step", "grad_bu")
    for i, mode in enumerate(("ticket", "dispatch", "auto", "dispatch", "ticket", "auto", "ticket")):
        monkeypatch.setenv("OSSM_SCAN_ORDER", mode)
        d = sets[i % 2]
        announce(f"runtime: scan order {mode} L={L} B={B} P={P} inputs {i % 2}")
        st = K.dlinoss_imex1_forward(*d["dev"])
        grads = K.dlinoss_imex1_backward(*d["dev"], st, d["go"])
        bseq = torch.view_as_real(d["dev"][3]).contiguous()
        y = K.lru_scan(d["lam"][0], d["lam"][1], bseq)
        r_st, r_grads, t_st, t_grads = d["truth"]
        assert_parity(to_np(st), r_st, t_st, RTOL, ATOL, f"{mode} states")
        for got, r32, r64, name in zip(grads, r_grads, t_grads, names):
            atol = ATOL if name == "grad_bu" else 2e-5 * max(1.0, float(np.abs(r64).max()))
            assert_parity(to_np(got), r32, r64, RTOL, atol, f"{mode} {name}")
        y = to_np(y)
        y = y[..., 0] + 1j * y[..., 1]
        assert_parity(y, d["lru"][0], d["lru"][1], RTOL, ATOL, f"{mode} lru")
    no_device_errors()


def test_scan_order_setting_is_checked(K, monkeypatch):
    """An OSSM_SCAN_ORDER other than auto, ticket or dispatch is refused with
    RuntimeError before anything is launched; forced dispatch order under
    stream capture is refused too (its tags are chosen on the host)."""
    a, g, dt, bu, _ = dlinoss_inputs(100, 2, 64, seed=53, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    K.dlinoss_imex1_forward(*args)
    monkeypatch.setenv("OSSM_SCAN_ORDER", "tickets")
    with pytest.raises(RuntimeError, match="OSSM_SCAN_ORDER"):
        K.dlinoss_imex1_forward(*args)
    monkeypatch.setenv("OSSM_SCAN_ORDER", "dispatch")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        K.dlinoss_imex1_forward(*args)  # eager warm-up of the side stream's scratch
    side.synchronize()
    graph = torch.cuda.CUDAGraph()
    announce("runtime: scan order setting checks")
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(RuntimeError, match="capture needs ticket order"):
                K.dlinoss_imex1_forward(*args)
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    monkeypatch.delenv("OSSM_SCAN_ORDER")
    st = K.dlinoss_imex1_forward(*args)
    assert_close(to_np(st), oracle.dlinoss_forward("imex1", a, g, dt, bu), RTOL, ATOL, "after refusals")
    no_device_errors()


def test_time_next_launch_records_kernel_events(K):
    """ossm_time_next_launch: the next D-LinOSS forward and backward kernels
    record the given events as their own start and end.  Each elapsed time is
    positive and below the whole call's wall time between host syncs; the
    outputs equal those of untimed calls to the usual run-to-run tolerance (the
    look-back may associate carries differently per run); a set timing is
    refused under stream capture
    (RuntimeError, nothing enqueued) and stays set for the next eager launch."""
    import ctypes
    import time

    from ossm_amd import _lib

    # the HIP runtime torch loaded (a second copy of the runtime must not load)
    lib = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
    hip = ctypes.CDLL(str(lib) if lib.exists() else "libamdhip64.so")
    evs = []
    for _ in range(4):
        e = ctypes.c_void_p()
        assert hip.hipEventCreate(ctypes.byref(e)) == 0
        evs.append(e)

    def elapsed(e0, e1):
        ms = ctypes.c_float()
        assert hip.hipEventElapsedTime(ctypes.byref(ms), e0, e1) == 0
        return ms.value

    L, B, P = 4096, 8, 128
    a, g, dt, bu, go = dlinoss_inputs(L, B, P, seed=51, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    god = to_dev(go)
    announce("runtime: time_next_launch")
    st_ref = K.dlinoss_imex1_forward(*args)
    gr_ref = K.dlinoss_imex1_backward(*args, st_ref, god)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    _lib.time_next_launch(evs[0].value, evs[1].value)
    st = K.dlinoss_imex1_forward(*args)
    _lib.time_next_launch(evs[2].value, evs[3].value)
    gr = K.dlinoss_imex1_backward(*args, st, god)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    f_ms, b_ms = elapsed(evs[0], evs[1]), elapsed(evs[2], evs[3])
    assert 0.0 < f_ms < wall_ms and 0.0 < b_ms < wall_ms, (f_ms, b_ms, wall_ms)
    st_np = to_np(st_ref)
    assert_close(to_np(st), st_np, RTOL, ATOL, "timed forward")
    for x, r, name in zip(gr, gr_ref, ("grad_a", "grad_g", "grad_step", "grad_bu")):
        rn = to_np(r)
        assert_close(to_np(x), rn, RTOL, 2e-5 * max(1.0, float(np.abs(rn).max())), name)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        K.dlinoss_imex1_forward(*args)  # the side stream's scratch exists
    side.synchronize()
    _lib.time_next_launch(evs[0].value, evs[1].value)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        graph.capture_begin()
        try:
            with pytest.raises(RuntimeError, match="under stream capture"):
                K.dlinoss_imex1_forward(*args)
        finally:
            graph.capture_end()
    torch.cuda.synchronize()
    st2 = K.dlinoss_imex1_forward(*args)  # takes the timing left set
    torch.cuda.synchronize()
    assert elapsed(evs[0], evs[1]) > 0.0
    assert_close(to_np(st2), st_np, RTOL, ATOL, "forward after the refused capture")
    no_device_errors()
    for e in evs:
        hip.hipEventDestroy(e)
