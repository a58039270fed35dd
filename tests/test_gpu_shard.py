"""GPU tests of the D-LinOSS forward split into time shards (ossm_amd.shard,
ossm_dlinoss_shard_carries / ossm_dlinoss_shard_fixup through the C ABI): each
shard scanned from a zero state, the carries between shards, each shard's
fix-up.  The result is compared with the oracle (fp32 reference, fp64 arbiter,
the north star's tolerance) and with one forward over the whole sequence."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle
from tests.gpu_util import (announce, assert_close, assert_parity, dlinoss_inputs, need_gpu,
                            no_device_errors, to_dev, to_np)

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


@pytest.fixture(scope="module")
def mods():
    need_gpu()
    from ossm_amd import _kernels, shard

    return _kernels, shard


def _truth(variant, a, g, dt, bu):
    ref = oracle.dlinoss_forward(variant, a, g, dt, bu)
    t64 = oracle.dlinoss_forward(variant, *(x.astype(np.float64) for x in (a, g, dt)),
                                 bu.astype(np.complex128))
    return ref, t64


# (L, B, P, shard lengths): one shard, equal shards, ragged shards (one step,
# lengths that end inside a sub-chunk), many shards
CASES = [(1000, 3, 70, [1000]), (1000, 3, 70, [500, 500]), (1000, 3, 70, [1, 313, 686]),
         (3001, 2, 96, [7, 1024, 1, 1500, 469]), (2048, 4, 64, [128] * 16)]


@pytest.mark.parametrize("variant", oracle.VARIANTS)
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sharded_forward_matches_oracle(mods, variant, case):
    K, shard = mods
    L, B, P, lengths = CASES[case]
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=70 + case, variant=variant)
    announce(f"shard {variant} L={L} B={B} P={P} shards={lengths}")
    st = to_np(shard.dlinoss_forward_sharded(variant, *(to_dev(x) for x in (a, g, dt, bu)), lengths))
    ref, t64 = _truth(variant, a, g, dt, bu)
    assert_parity(st, ref, t64, RTOL, ATOL, "sharded states")
    whole = to_np(getattr(K, f"dlinoss_{variant}_forward")(*(to_dev(x) for x in (a, g, dt, bu))))
    assert_parity(st, whole, t64, RTOL, ATOL, "sharded vs whole")
    no_device_errors()


def test_sharded_forward_config2_eight_shards(mods):
    """Config 2 (B=32, L=4096, P=128) in eight shards of 512 steps: the states
    of one forward over the whole sequence, elementwise."""
    K, shard = mods
    L, B, P = 4096, 32, 128
    a, g, dt, bu, _ = dlinoss_inputs(L, B, P, seed=77, variant="imex1")
    announce("shard imex1 config 2, 8 shards")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    st = to_np(shard.dlinoss_forward_sharded("imex1", *args, [512] * 8))
    ref, t64 = _truth("imex1", a, g, dt, bu)
    assert_parity(st, ref, t64, RTOL, ATOL, "config 2 sharded states")
    no_device_errors()


def test_shard_entry_points_check_their_arguments(mods):
    """Shard lengths that do not sum to L, an empty shard, too many shards and
    an unknown variant are refused before anything is launched."""
    K, shard = mods
    from ossm_amd import _lib

    lib = _lib.load()
    a, g, dt, bu, _ = dlinoss_inputs(100, 2, 8, seed=78, variant="imex1")
    args = [to_dev(x) for x in (a, g, dt, bu)]
    announce("shard argument checks")
    with pytest.raises(ValueError, match="sum to L"):
        shard.dlinoss_forward_sharded("imex1", *args, [50, 49])
    with pytest.raises(ValueError, match="Unknown D-LinOSS variant"):
        shard.dlinoss_forward_sharded("rk4", *args, [100])
    states = torch.zeros((100, 2, 8, 2), dtype=torch.complex64, device="cuda")
    carries = torch.zeros((65, 2, 8, 2), dtype=torch.complex64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    ptrs = [t.data_ptr() for t in args[:3]]
    for lengths, n, what in (([60, 40], 2, None), ([60, 39], 2, "sum to"), ([100, 0], 2, "at least one"),
                             ([1] * 65, 65, "n_shards")):
        arr = (ctypes.c_int64 * len(lengths))(*lengths)
        rc = lib.ossm_dlinoss_shard_carries(0, *ptrs, states.data_ptr(), 100, arr, n,
                                            carries.data_ptr(), 2, 8, stream)
        if what is None:
            assert rc == 0
        else:
            assert rc == 1 and what in lib.ossm_last_error().decode()
    assert lib.ossm_dlinoss_shard_fixup(7, *ptrs, carries.data_ptr(), states.data_ptr(), 100, 2, 8,
                                        stream) == 1
    torch.cuda.synchronize()
    # the carries of all-zero states are zero
    assert_close(to_np(carries[:2]), np.zeros((2, 2, 8, 2), np.complex64), 0, 0, "zero carries")
    no_device_errors()
