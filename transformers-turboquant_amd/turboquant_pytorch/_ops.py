"""torch.ops.tq: the PyTorch-ROCm operator layer over libtq_amd.so's C ABI.

``_tq_torch.so`` (built from csrc/tq_torch.cpp next to libtq_amd.so) registers
one op per C entry point.  The ops allocate their outputs with torch and launch
on torch's current stream, so the product path calls them directly; the ctypes
binding in ``_native`` is kept for calling the C ABI itself (its tests, and the
binding a reference-side caller would write).  For tensors on a GPU the
extension is mandatory: :func:`ops` raises if it is missing.
"""

from __future__ import annotations

import os
import threading

import torch

_OPS_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_tq_torch.so")
_lock = threading.Lock()
_loaded = False


def library_path() -> str:
    return _OPS_PATH


def ops():
    """The ``torch.ops.tq`` namespace, loading the extension on first use."""
    global _loaded
    if not _loaded:
        with _lock:
            if not _loaded:
                if not os.path.exists(_OPS_PATH):
                    raise RuntimeError(
                        f"TurboQuant torch extension not built: {_OPS_PATH} is missing. "
                        "Run `python -c 'import __graft_entry__ as g; g.build()'` "
                        "or `make -C transformers-turboquant_amd/csrc`.")
                torch.ops.load_library(_OPS_PATH)
                _loaded = True
    return torch.ops.tq
