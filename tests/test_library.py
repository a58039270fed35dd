"""CPU-side checks of the boundary: the C-ABI library loads and exports every
symbol include/ossm_scan.h declares, and the drop-in module exposes every
name of the reference's ``ossm._kernels`` (bindings.cpp:159-224).  No
compute call is made (there is no GPU here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "ossm_scan.h"

# every Python-visible name of the reference extension module
REFERENCE_NAMES = (
    [f"dlinoss_{v}_{d}" for v in ("imex1", "imex2", "im", "ex") for d in ("forward", "backward")]
    + [f"sdlinoss_{v}_{d}" for v in ("imex1", "imex2", "im", "ex") for d in ("forward", "backward")]
    + ["linoss_scan", "lru_scan", "s5_scan", "linear_rnn_scan", "selective_scan",
       "selective_scan_backward", "selective_scan_cuda", "selective_scan_cuda_backward"]
)


def _declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ossm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("ossm_dlinoss_forward", "ossm_dlinoss_backward", "ossm_linoss_forward",
              "ossm_linoss_backward", "ossm_selective_forward", "ossm_selective_backward",
              "ossm_selective_num_chunks", "ossm_abi_version", "ossm_last_error",
              "ossm_device_error_bits", "ossm_selective_forward_bf16",
              "ossm_selective_backward_bf16", "ossm_sdlinoss_forward", "ossm_sdlinoss_backward",
              "ossm_sdlinoss_forward_f64", "ossm_sdlinoss_backward_f64",
              "ossm_linoss_forward_f64", "ossm_linoss_backward_f64", "ossm_dlinoss_forward_f64",
              "ossm_dlinoss_backward_f64",
              "ossm_diag_scan_forward", "ossm_diag_scan_backward", "ossm_diag_scan_forward_f64",
              "ossm_diag_scan_backward_f64", "ossm_dlinoss_layer_forward", "ossm_dlinoss_layer_backward",
              "ossm_selective_mamba_forward", "ossm_selective_mamba_backward",
              "ossm_mamba_conv_forward", "ossm_mamba_conv_backward", "ossm_time_next_launch",
              "ossm_selective_forward_skip", "ossm_selective_backward_skip",
              "ossm_dlinoss_shard_carries", "ossm_dlinoss_shard_fixup"):
        assert n in names, n


def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (binds the HIP runtime first, as the product does)

    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in _declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # every declared symbol has a ctypes signature in the binding
    assert set(_declared_functions()) == set(_lib.EXPORTED)
    assert _lib.load().ossm_abi_version() == 16


def test_selective_skip_entry_points_refuse_a_null_d():
    """The skip entry points check their own arguments before any HIP call."""
    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    lib = _lib.load()
    p = ctypes.c_void_p(256)  # never dereferenced: the calls fail first
    assert lib.ossm_selective_forward_skip(0, p, p, p, p, p, None, None, p, p, p, 1, 1, 1, 1, None) == 1
    assert b"null skip D" in lib.ossm_last_error()
    assert lib.ossm_selective_backward_skip(0, p, p, p, p, p, p, p, None, p, p, p, p, p, p, p, None,
                                            None, 1, 1, 1, 1, None) == 1
    assert b"null skip D or dD" in lib.ossm_last_error()


def test_shard_entry_points_check_shard_lengths_before_any_hip_call():
    """ossm_dlinoss_shard_carries refuses shard counts outside 1..64, empty
    shards and lengths that do not sum to the states' length, and both shard
    entry points refuse negative sizes, all before any HIP call."""
    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    lib = _lib.load()
    p = ctypes.c_void_p(256)  # never dereferenced: the calls fail first

    def carries(lengths, n, L):
        arr = (ctypes.c_int64 * max(1, len(lengths)))(*lengths)
        return lib.ossm_dlinoss_shard_carries(0, p, p, p, p, L, arr, n, p, 2, 8, None)

    assert carries([], 0, 10) == 1 and b"n_shards" in lib.ossm_last_error()
    assert carries([1] * 65, 65, 65) == 1 and b"n_shards" in lib.ossm_last_error()
    assert carries([5, 0, 5], 3, 10) == 1 and b"at least one step" in lib.ossm_last_error()
    assert carries([5, 4], 2, 10) == 1 and b"sum to 9" in lib.ossm_last_error()
    assert carries([5, 5], 2, -1) == 1 and b"negative size" in lib.ossm_last_error()
    assert lib.ossm_dlinoss_shard_fixup(0, p, p, p, p, p, -1, 2, 8, None) == 1
    assert b"negative size" in lib.ossm_last_error()


def test_time_next_launch_argument_checks():
    """The measurement hook takes both events or neither; it makes no HIP call
    when set, so it runs here."""
    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    lib = _lib.load()
    assert lib.ossm_time_next_launch(None, ctypes.c_void_p(16)) == 1  # OSSM_ERR_INVALID_ARGUMENT
    assert b"both events or neither" in lib.ossm_last_error()
    assert lib.ossm_time_next_launch(None, None) == 0
    with pytest.raises(RuntimeError, match="both events or neither"):
        _lib.time_next_launch(16, None)


def test_dropin_module_has_every_reference_name():
    from ossm_amd import _kernels

    for name in REFERENCE_NAMES:
        assert callable(getattr(_kernels, name)), name


def test_cpu_tensors_without_delegate_raise_runtime_error():
    import torch

    from ossm_amd import _kernels

    _kernels.set_cpu_delegate(None)
    a = torch.ones(3)
    bu = torch.zeros(4, 2, 3, dtype=torch.complex64)
    with pytest.raises(RuntimeError, match="CPU tensors"):
        _kernels.dlinoss_imex1_forward(a, a, a, bu)
    with pytest.raises(RuntimeError, match="bu must have shape"):
        _kernels.dlinoss_imex1_forward(a, a, a, bu[0])
    with pytest.raises(RuntimeError):
        _kernels.lru_scan(torch.ones(3), torch.ones(3), torch.zeros(4, 2, 3, 2))


def test_cpu_delegate_routes_to_the_reference_module():
    """With the reference's CPU build attached (oracle/_ref, when built), CPU
    calls return the reference's own results."""
    import numpy as np
    import torch

    import oracle
    from ossm_amd import _kernels

    ref = oracle.reference_module()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    _kernels.set_cpu_delegate(ref)
    try:
        rng = np.random.default_rng(0)
        a = torch.tensor(rng.uniform(0.1, 1, 5), dtype=torch.float32)
        g = torch.tensor(rng.uniform(0, 1, 5), dtype=torch.float32)
        dt = torch.tensor(rng.uniform(0.1, 0.9, 5), dtype=torch.float32)
        bu = torch.tensor(rng.normal(size=(7, 2, 5)) + 1j * rng.normal(size=(7, 2, 5)),
                          dtype=torch.complex64)
        got = _kernels.dlinoss_im_forward(a, g, dt, bu)
        assert torch.equal(got, ref.dlinoss_im_forward(a, g, dt, bu))
    finally:
        _kernels.set_cpu_delegate(None)


# the reference's operator schemas (_dlinoss_scan.py:183-206)
_REF_FWD_SCHEMA = "ossm::dlinoss_{v}_forward(Tensor a_diag, Tensor g_diag, Tensor step, Tensor bu) -> Tensor"
_REF_BWD_SCHEMA = ("ossm::dlinoss_{v}_backward(Tensor a_diag, Tensor g_diag, Tensor step, Tensor bu, "
                   "Tensor states, Tensor grad_output) -> (Tensor, Tensor, Tensor, Tensor)")


@pytest.mark.parametrize("variant", ["imex1", "imex2", "im", "ex"])
def test_torch_library_ops_schema_and_meta(variant):
    """The ``ossm::dlinoss_*`` operators carry the reference's schemas, and
    their Meta implementations give outputs of the kernels' shapes and dtypes
    (states [L, B, P, 2] like bu; gradients like a, g, step and bu)."""
    import torch

    from ossm_amd import _lib, bridge

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    assert bridge.CUSTOM_OPS
    fwd = getattr(torch.ops.ossm, f"dlinoss_{variant}_forward")
    bwd = getattr(torch.ops.ossm, f"dlinoss_{variant}_backward")
    assert str(fwd.default._schema) == _REF_FWD_SCHEMA.format(v=variant)
    assert str(bwd.default._schema) == _REF_BWD_SCHEMA.format(v=variant)
    a = torch.empty(5, device="meta")
    bu = torch.empty(7, 3, 5, dtype=torch.complex64, device="meta")
    st = fwd(a, a, a, bu)
    assert st.shape == (7, 3, 5, 2) and st.dtype == torch.complex64 and st.device.type == "meta"
    grads = bwd(a, a, a, bu, st, bu)
    assert [tuple(g.shape) for g in grads] == [(5,), (5,), (5,), (7, 3, 5)]
    assert [g.dtype for g in grads] == [torch.float32] * 3 + [torch.complex64]


@pytest.mark.parametrize("shape", [(4096, 64, 160), (65536, 4, 256), (2**25 + 1, 1, 1)],
                         ids=lambda s: "x".join(map(str, s)))
def test_noalloc_forward_refuses_above_its_limit_on_the_host(shape):
    """ossm_dlinoss_forward_noalloc serves at most 33,554,432 state-steps
    (L*B*P) per call, whatever tile the allocating forward picks for that
    shape; above it the call returns OSSM_ERR_UNSUPPORTED from its host-side
    checks, before any HIP call, so the pointers (host dummies here, no GPU)
    are never read."""
    import torch  # noqa: F401  (binds the HIP runtime first, as the product does)

    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    f = lib.ossm_dlinoss_forward_noalloc
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 5 + [ctypes.c_int64] * 3 + [ctypes.c_void_p]
    lib.ossm_last_error.restype = ctypes.c_char_p
    buf = ctypes.create_string_buffer(16)
    p = ctypes.addressof(buf)
    L, B, P = shape
    assert L * B * P > 2**25
    assert f(0, p, p, p, p, p, L, B, P, None) == 3  # OSSM_ERR_UNSUPPORTED
    assert b"33,554,432" in lib.ossm_last_error()


def test_sharded_forward_checks_its_arguments_on_the_host():
    """ossm_amd.shard refuses an unknown variant and host tensors before it
    reaches the library (no GPU needed)."""
    import torch

    from ossm_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libossm_scan.so not built (python -m ossm_amd.build)")
    from ossm_amd import shard

    p = torch.zeros(4)
    bu = torch.zeros((8, 2, 4), dtype=torch.complex64)
    with pytest.raises(ValueError, match="Unknown D-LinOSS variant"):
        shard.dlinoss_forward_sharded("rk4", p, p, p, bu, [8])
    with pytest.raises(RuntimeError, match="device tensor"):
        shard.dlinoss_forward_sharded("imex1", p, p, p, bu, [4, 4])
