"""Write kv_format_v1.safetensors: a tiny turboquant-kv container that pins the format.

    python tests/golden/make_kv_format.py

Two groups with deterministic contents (see `planes()`): "p" in the packed layout
(B1 H2 S3 D32, key bits 3, value bits 3, seeds 7 / 10007, keys and values) and "u"
in the unpacked layout (keys only).  tests/test_serialize_cpu.py reads it back and
checks every plane and metadata field, so a change to the writer or reader that
alters the format fails there.
"""

import os
import sys

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "transformers-turboquant_amd"))

from turboquant_pytorch.serialize import save_groups  # noqa: E402

B, H, S, D = 1, 2, 3, 32
N = B * H * S


def _bytes(n, cols, mul, add):
    return ((torch.arange(n * cols) * mul + add) % 256).to(torch.uint8).reshape(n, cols)


def _halves(n, base):
    return (torch.arange(n, dtype=torch.float32) * 0.25 + base).to(torch.float16)


def planes():
    """The fixture's groups, as save_groups takes them."""
    pk = {"packed_key_indices": _bytes(N, 8, 37, 11), "packed_qjl_signs": _bytes(N, 4, 59, 3),
          "residual_norm": _halves(N, 0.5).reshape(B, H, S), "vec_norms": _halves(N, 2.0).reshape(B, H, S),
          "shape": (B, H, S, D)}
    pv = {"packed_indices": _bytes(N, 12, 101, 17), "vec_norms": _halves(N, 4.0), "shape": (B, H, S, D)}
    k_mse = ((torch.arange(N * D, dtype=torch.float32) % 97) / 16 - 3).to(torch.float16).reshape(B, H, S, D)
    signs = torch.where(torch.arange(N * D) % 3 == 0, 1, -1).to(torch.int8).reshape(B, H, S, D)
    uk = {"k_mse": k_mse, "qjl_signs": signs, "residual_norm": _halves(N, 1.0).reshape(B, H, S),
          "shape": (B, H, S, D)}
    return [{"name": "p", "keys": pk, "values": pv, "key_bits": 3, "value_bits": 3, "key_seed": 7,
             "value_seed": 10007},
            {"name": "u", "keys": uk, "values": None, "key_bits": 3, "key_seed": 7}]


if __name__ == "__main__":
    save_groups(os.path.join(HERE, "kv_format_v1.safetensors"), planes(), metadata={"note": "format fixture"})
