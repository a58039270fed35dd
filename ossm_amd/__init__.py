"""ossm_amd — MI355X (gfx950) scan kernels behind the ``ossm._kernels`` interface.

``ossm_amd._kernels`` is the drop-in module (same names and signatures as the
reference extension); ``ossm_amd.bridge`` holds autograd wrappers with the
reference bridges' semantics; the C ABI is ``include/ossm_scan.h``, built by
``python -m ossm_amd.build`` into ``ossm_amd/_lib/libossm_scan.so``.
"""

from __future__ import annotations

import sys
import types


def install_as_ossm_kernels() -> types.ModuleType:
    """Register this library as ``ossm._kernels`` so the reference's Python
    package picks it up on import (``from ossm import _kernels``)."""
    from . import _kernels

    sys.modules["ossm._kernels"] = _kernels
    parent = sys.modules.get("ossm")
    if parent is not None:
        setattr(parent, "_kernels", _kernels)
    return _kernels


__all__ = ["install_as_ossm_kernels"]
