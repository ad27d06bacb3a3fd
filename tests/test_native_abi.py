"""The C-ABI library loads and exports every entry point declared in include/tq_api.h.

No kernel is launched here: only argument validation, which returns before any
HIP call.
"""

import os
import re
import subprocess

import pytest

from turboquant_pytorch import _native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _declared():
    text = open(os.path.join(ROOT, "include", "tq_api.h")).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(tq_\w+)\s*\(", text, re.M)))


def test_header_declarations_are_bound():
    assert _declared() == sorted(_native.EXPORTED)


def test_library_exports_every_symbol():
    path = _native.library_path()
    assert os.path.exists(path), "build the library first (__graft_entry__.build())"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (tq_\w+)", out))
    missing = set(_declared()) - exported
    assert not missing, missing


def test_argument_validation_without_gpu():
    lib = _native.lib()
    assert lib.tq_version() >= 100
    assert lib.tq_out_cols(128, 3) == 48 and lib.tq_out_cols(7, 3) == 3
    assert lib.tq_pack_bits(None, 4, 128, 128, 9, None, 144, None) == -1
    assert b"between 1 and 8" in lib.tq_last_error()
    assert lib.tq_compress_keys(None, 0, 1, 1, 1, 100, 0, 0, 0, None, None, None, None, 2,
                                None, None, None, None, None, None, None) == -2
    assert b"head_dim 100" in lib.tq_last_error()
    assert lib.tq_compress_keys(None, 0, 1, 1, 1, 264, 0, 0, 0, None, None, None, None, 2,
                                None, None, None, None, None, None, None) == -2
    assert lib.tq_attention_fwd(*([None] * 7), 5, None, None, None, 3, None, 1, 8, 8, 1, 1, 128, 0.0, 1.0, 0,
                                None, 0, 0, 0, 0, None, 0, 0, 0, 0, None, 0, None) == -1
    assert b"key bits" in lib.tq_last_error()
    # split-K workspace: the decode kernels' partials (head_dim 64 / 128, <= 16 columns per kv
    # head), or the tiled kernel split over keys (any head dim, the kv head's columns in one query
    # block, at least 512 keys): B * Hkv * splits * columns * (row floats + 2) * 4 bytes, with
    # about 512 blocks of >= 256 keys (whole 32-key tiles) and rows of 64 / 128 / 256 floats
    assert lib.tq_attention_workspace_size(4, 32, 8, 1, 32768, 128, 3) > 0

    def tiled(B, Hq, Hkv, Sq, Sk, d):
        groups = B * Hkv
        ns = min(-(-512 // groups), Sk // 256, 1024)
        chunk = -(-(-(-Sk // ns)) // 32) * 32
        ns = -(-Sk // chunk)
        rowf = 64 if -(-d // 32) * 32 <= 64 else (128 if -(-d // 32) * 32 <= 128 else 256)
        return groups * ns * (Hq // Hkv) * Sq * (rowf + 2) * 4

    assert lib.tq_attention_workspace_size(4, 32, 8, 8, 32768, 128, 3) == tiled(4, 32, 8, 8, 32768, 128)
    assert lib.tq_attention_workspace_size(4, 32, 8, 1, 32768, 96, 3) == tiled(4, 32, 8, 1, 32768, 96)
    assert lib.tq_attention_workspace_size(4, 32, 8, 5, 32768, 64, 3) == tiled(4, 32, 8, 5, 32768, 64)
    assert lib.tq_attention_workspace_size(4, 32, 8, 3, 32768, 64, 4) >= tiled(4, 32, 8, 3, 32768, 64)
    assert lib.tq_attention_workspace_size(4, 32, 8, 1, 32768, 64, 3) >= tiled(4, 32, 8, 1, 32768, 64)
    assert lib.tq_attention_workspace_size(1, 12, 12, 1, 5000, 96, 2) == tiled(1, 12, 12, 1, 5000, 96)
    assert lib.tq_attention_workspace_size(2, 8, 2, 1, 400, 96, 3) == 0       # too few keys to split
    assert lib.tq_attention_workspace_size(2, 8, 2, 1, 400, 64, 3) > 0        # the decode kernels' partials
    assert lib.tq_attention_workspace_size(1, 256, 1, 1, 32768, 64, 3) == 0   # group beyond one block
    with pytest.raises(RuntimeError, match="group size|multiple"):
        _native.check(lib.tq_attention_scores(*([None] * 7), 1, 6, 4, 1, 1, 128, 3, 0.0, None, None),
                      "scores")


def test_missing_library_fails_loudly(monkeypatch):
    """With the shared library absent the GPU path raises; nothing falls back to the CPU."""
    monkeypatch.setattr(_native, "_LIB_PATH", os.path.join(ROOT, "no_such_dir", "libtq_amd.so"))
    monkeypatch.setattr(_native, "_lib", None)
    with pytest.raises(RuntimeError, match="not built"):
        _native.lib()


OPS = ("pack_bits", "unpack_bits", "quantize_pack", "dequantize", "compress_keys", "compress_values",
       "decompress_values", "query_prep", "scores", "attention", "workspace_size")


def test_torch_extension_registers_every_op():
    """torch.ops.tq (csrc/tq_torch.cpp) loads without a GPU and registers one op per C entry
    point the product path calls; with CPU tensors the GPU ops refuse to run."""
    import torch

    from turboquant_pytorch import _ops

    tq = _ops.ops()
    for name in OPS:
        assert hasattr(tq, name), name
    assert "int workspace" in str(tq.attention.default._schema)
    with pytest.raises(NotImplementedError):
        tq.pack_bits(torch.zeros(2, 8, dtype=torch.int32), 3)


def test_missing_extension_raises(monkeypatch):
    from turboquant_pytorch import _ops

    monkeypatch.setattr(_ops, "_OPS_PATH", os.path.join(ROOT, "no_such_dir", "_tq_torch.so"))
    monkeypatch.setattr(_ops, "_loaded", False)
    with pytest.raises(RuntimeError, match="not built"):
        _ops.ops()
