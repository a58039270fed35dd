"""Loader for libossm_scan.so (the C ABI declared in include/ossm_scan.h).

torch is imported first so that the HIP runtime torch ships (SONAME
libamdhip64.so.7) is the one the library binds to: streams handed over from
torch are then valid in the library.  A missing library is an ImportError —
there is no fallback path behind this module.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch  # noqa: F401  (must precede the library load)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libossm_scan.so"

_c_int64 = ctypes.c_int64
_vp = ctypes.c_void_p
_fp = ctypes.c_void_p  # float* passed as raw device addresses
_dp = ctypes.c_void_p  # double* passed as raw device addresses

_SIGNATURES = {
    "ossm_abi_version": (ctypes.c_int, []),
    "ossm_test_skew_tickets": (ctypes.c_int, [_vp, ctypes.c_uint64]),
    "ossm_time_next_launch": (ctypes.c_int, [_vp, _vp]),
    "ossm_last_error": (ctypes.c_char_p, []),
    "ossm_device_error_bits": (ctypes.c_uint32, [_vp]),
    "ossm_dlinoss_forward": (
        ctypes.c_int, [ctypes.c_int, _fp, _fp, _fp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_forward_noalloc": (
        ctypes.c_int, [ctypes.c_int, _fp, _fp, _fp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_backward": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _fp, _fp, _vp, _vp, _vp, _fp, _fp, _fp, _vp, _c_int64, _c_int64,
         _c_int64, _vp]),
    "ossm_linoss_forward": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_linoss_backward": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_num_chunks": (ctypes.c_int64, [_c_int64]),
    "ossm_selective_forward": (
        ctypes.c_int,
        [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_backward": (
        ctypes.c_int,
        [_fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _c_int64,
         _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_sdlinoss_forward": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64,
         _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_sdlinoss_backward": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64,
         _vp, _vp, _vp, _fp, _fp, _fp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_forward_f64": (
        ctypes.c_int, [ctypes.c_int, _dp, _dp, _dp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_backward_f64": (
        ctypes.c_int,
        [ctypes.c_int, _dp, _dp, _dp, _vp, _vp, _vp, _dp, _dp, _dp, _vp, _c_int64, _c_int64,
         _c_int64, _vp]),
    "ossm_linoss_forward_f64": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_linoss_backward_f64": (
        ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_sdlinoss_forward_f64": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64,
         _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_sdlinoss_backward_f64": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64, _fp, _c_int64, _c_int64,
         _vp, _vp, _vp, _fp, _fp, _fp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_forward_bf16": (
        ctypes.c_int,
        [_vp, _vp, _fp, _vp, _vp, _vp, _vp, _vp, _fp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_backward_bf16": (
        ctypes.c_int,
        [_vp, _vp, _vp, _fp, _vp, _vp, _vp, _fp, _vp, _vp, _vp, _fp, _vp, _vp, _vp, _c_int64,
         _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_forward_skip": (
        ctypes.c_int,
        [ctypes.c_int, _vp, _vp, _fp, _vp, _vp, _fp, _vp, _vp, _vp, _fp, _c_int64, _c_int64,
         _c_int64, _c_int64, _vp]),
    "ossm_selective_backward_skip": (
        ctypes.c_int,
        [ctypes.c_int, _vp, _vp, _vp, _fp, _vp, _vp, _fp, _vp, _fp, _vp, _vp, _vp, _fp, _vp, _vp,
         _fp, _vp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_diag_scan_forward": (
        ctypes.c_int, [_fp, _fp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_diag_scan_backward": (
        ctypes.c_int, [_fp, _fp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_diag_scan_forward_f64": (
        ctypes.c_int, [_fp, _fp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_diag_scan_backward_f64": (
        ctypes.c_int, [_fp, _fp, _vp, _vp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_layer_forward": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _vp, _c_int64, _c_int64, _c_int64,
         _c_int64, _vp]),
    "ossm_dlinoss_layer_backward": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _vp, _fp, _vp, _vp, _fp, _fp, _fp,
         _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_mamba_forward": (
        ctypes.c_int,
        [_fp, _c_int64, _fp, _c_int64, _fp, _fp, _fp, _fp, _c_int64, _fp, _c_int64, _fp, _fp, _fp,
         _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_selective_mamba_backward": (
        ctypes.c_int,
        [_fp, _fp, _c_int64, _fp, _c_int64, _fp, _fp, _fp, _fp, _c_int64, _fp, _c_int64, _fp, _fp,
         _fp, _fp, _fp, _fp, _fp, _fp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_shard_carries": (
        ctypes.c_int,
        [ctypes.c_int, _fp, _fp, _fp, _vp, _c_int64, _vp, ctypes.c_int, _vp, _c_int64, _c_int64, _vp]),
    "ossm_dlinoss_shard_fixup": (
        ctypes.c_int, [ctypes.c_int, _fp, _fp, _fp, _vp, _vp, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_mamba_conv_forward": (
        ctypes.c_int, [_fp, _c_int64, _fp, _fp, _fp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
    "ossm_mamba_conv_backward": (
        ctypes.c_int,
        [_fp, _c_int64, _fp, _fp, _fp, _fp, _fp, _fp, _c_int64, _c_int64, _c_int64, _c_int64, _vp]),
}

EXPORTED = tuple(_SIGNATURES)

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Load the library once; ImportError if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m ossm_amd.build` "
                "(the HIP path has no fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


# OSSM_CHECK_DEVICE_ERRORS=1: after every successful call made outside stream
# capture, synchronise the current stream and raise RuntimeError if a kernel
# raised a protocol error bit (a look-back wait that gave up, an out-of-range
# ticket).  Off by default: the check costs a stream synchronisation per call.
CHECK_DEVICE_ERRORS = os.environ.get("OSSM_CHECK_DEVICE_ERRORS", "0") not in ("", "0")


def check(rc: int) -> None:
    """Raise RuntimeError (the reference's TORCH_CHECK surface) on a nonzero status.
    Called inside the ``torch.cuda.device`` block of the call it checks."""
    if rc != 0:
        msg = load().ossm_last_error().decode(errors="replace")
        raise RuntimeError(msg or f"ossm_scan call failed with status {rc}")
    # not under stream capture: the check synchronises the stream and copies
    # the bits to the host, which a capture cannot record (it would invalidate it)
    if CHECK_DEVICE_ERRORS and not torch.cuda.is_current_stream_capturing():
        bits = device_error_bits()
        if bits:
            raise RuntimeError(f"ossm_scan: a kernel raised device error bits {bits:#x} "
                               "(1 = look-back wait gave up, 2 = out-of-range ticket); "
                               "its outputs are not valid")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def device_error_bits(device: Optional[torch.device] = None) -> int:
    """Synchronise the current stream and return (and clear) its kernel error bits."""
    dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
    with torch.cuda.device(dev):
        return int(load().ossm_device_error_bits(torch.cuda.current_stream(dev).cuda_stream))


def time_next_launch(start_event: Optional[int], stop_event: Optional[int]) -> None:
    """The next LinOSS / D-LinOSS scan kernel this thread launches records these
    two hipEvent_t handles as its own start and end (no event packets between
    kernels); two Nones clear the setting."""
    check(load().ossm_time_next_launch(start_event, stop_event))
