"""Sequence (context-parallel) sharding of the D-LinOSS forward, run on one GPU.

On G GPUs each would scan its own span of the sequence from a zero state, the
carries entering the spans would be an exclusive scan over the GPUs of one
affine map per channel (M^len, last zero-start state), and each GPU would then
correct its span with a fix-up pass.  ``dlinoss_forward_sharded`` runs those
three steps on one device, in shard order, through the library's C ABI:
``ossm_dlinoss_forward`` per shard, ``ossm_dlinoss_shard_carries`` for the
scan over shards and ``ossm_dlinoss_shard_fixup`` per shard.  Its result equals
one ``dlinoss_<v>_forward`` over the whole sequence to rounding.  The
reference has no counterpart (it scans each sequence in one piece).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib

_VARIANTS = {"imex1": 0, "imex2": 1, "im": 2, "ex": 3}


def _check_inputs(a_diag, g_diag, step, bu):
    if not bu.is_cuda:
        raise RuntimeError("dlinoss_forward_sharded: bu must be a device tensor")
    if bu.dim() != 3 or bu.dtype != torch.complex64:
        raise RuntimeError("dlinoss_forward_sharded: bu must be complex64 [L, B, P]")
    P = bu.size(2)
    for name, t in (("a_diag", a_diag), ("g_diag", g_diag), ("step", step)):
        if t.dtype != torch.float32 or t.numel() != P or t.device != bu.device:
            raise RuntimeError(f"dlinoss_forward_sharded: {name} must be float32 [P] on bu's device")


def dlinoss_forward_sharded(variant: str, a_diag, g_diag, step, bu,
                            shard_lengths: Sequence[int]) -> torch.Tensor:
    """The D-LinOSS forward of ``bu [L, B, P]`` computed in len(shard_lengths)
    consecutive time shards: each from a zero state, then the carries between
    shards, then each shard's fix-up.  Returns ``states [L, B, P, 2]``."""
    if variant not in _VARIANTS:
        raise ValueError(f"Unknown D-LinOSS variant {variant!r}")
    _check_inputs(a_diag, g_diag, step, bu)
    L, B, P = bu.shape
    lengths = [int(n) for n in shard_lengths]
    if any(n < 1 for n in lengths) or sum(lengths) != L:
        raise ValueError(f"shard lengths {lengths} must be positive and sum to L = {L}")
    v = _VARIANTS[variant]
    a, g, s = (t.contiguous() for t in (a_diag, g_diag, step))
    bu = bu.contiguous()
    lib = _lib.load()
    states = torch.empty((L, B, P, 2), dtype=torch.complex64, device=bu.device)
    carries = torch.empty((len(lengths), B, P, 2), dtype=torch.complex64, device=bu.device)
    starts = [sum(lengths[:k]) for k in range(len(lengths))]
    with torch.cuda.device(bu.device):
        stream = _lib.stream_of(bu)
        for t0, n in zip(starts, lengths):  # each shard from a zero state
            _lib.check(lib.ossm_dlinoss_forward(v, a.data_ptr(), g.data_ptr(), s.data_ptr(),
                                                bu[t0:t0 + n].data_ptr(), states[t0:t0 + n].data_ptr(),
                                                n, B, P, stream))
        arr = (ctypes.c_int64 * len(lengths))(*lengths)
        _lib.check(lib.ossm_dlinoss_shard_carries(v, a.data_ptr(), g.data_ptr(), s.data_ptr(),
                                                  states.data_ptr(), L, arr, len(lengths),
                                                  carries.data_ptr(), B, P, stream))
        for k, (t0, n) in enumerate(zip(starts, lengths)):
            if k == 0:
                continue  # the first shard starts from the true (zero) state
            _lib.check(lib.ossm_dlinoss_shard_fixup(v, a.data_ptr(), g.data_ptr(), s.data_ptr(),
                                                    carries[k].data_ptr(),
                                                    states[t0:t0 + n].data_ptr(), n, B, P, stream))
    return states
