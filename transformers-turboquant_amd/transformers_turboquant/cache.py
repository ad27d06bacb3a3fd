"""Compressed KV cache for incremental decoding.

The reference recomputes every forward from the full sequence and disables the
cache (patch.py:81); a compressed cache exists there only as a tensor-level
sketch (turboquant.py:199-286, ``TurboQuantKVCache``).  ``TurboQuantCache``
stores what the patched attention layers compress, so each decoding step
compresses only its new tokens and attends to everything cached:

* GPU: per layer, the packed planes of ``capacity`` positions per (batch, kv
  head) — key codes, QJL signs, residual and vector norms, value codes and
  norms — laid out ``[B, Hkv, capacity, ...]``.  New tokens are compressed and
  copied into positions ``[length, length + S)``; capacity grows by doubling.
  Attention reads the first ``length`` rows of each plane in place (the
  ``kv_stride`` entry of the dicts, see ``tq_attention_fwd_kv``), so the
  split-K decode kernels stream exactly the cached bytes.
* CPU: the reference's unpacked formats, concatenated along the sequence.

Pass an instance to ``generate(..., past_key_values=TurboQuantCache(),
use_cache=True)`` on a model patched by ``apply_turboquant``.
"""

from __future__ import annotations

import math

import torch
from transformers.cache_utils import Cache, CacheLayerMixin

__all__ = ["TurboQuantCache", "TurboQuantCacheLayer"]

_KEY_PLANES = ("packed_key_indices", "packed_qjl_signs", "residual_norm", "vec_norms")
_VAL_PLANES = ("packed_indices", "vec_norms")
_ROUND = 256  # capacity granularity (positions)


class TurboQuantCacheLayer(CacheLayerMixin):
    """One attention layer's compressed keys and values."""

    is_compileable = False
    supports_early_init = False

    def __init__(self, **kwargs):
        super().__init__()
        self.length = 0
        self.capacity = 0
        self.shape: tuple | None = None  # (B, Hkv, D)
        self.kp: dict[str, torch.Tensor] | None = None  # GPU key planes [B, Hkv, capacity, ...]
        self.vp: dict[str, torch.Tensor] | None = None  # GPU value planes
        self.cpu_k: dict | None = None  # CPU unpacked dicts
        self.cpu_v: dict | None = None
        self.codec: dict = {}  # key/value bits and seeds of the compressors that filled the layer

    # ------------------------------------------------------------------ Cache layer API
    def lazy_initialization(self, key_states, value_states) -> None:
        return None

    def update(self, key_states, value_states, *args, **kwargs):
        raise NotImplementedError(
            "TurboQuantCache holds compressed planes; it is filled by attention modules patched with "
            "apply_turboquant, not by uncompressed key/value updates")

    def get_seq_length(self) -> int:
        return self.length

    def get_mask_sizes(self, query_length: int) -> tuple[int, int]:
        return self.length + query_length, 0

    def get_max_length(self) -> int:
        return -1

    def reset(self) -> None:
        self.length = 0
        self.cpu_k = self.cpu_v = None

    def crop(self, tokens_to_remove: int) -> None:
        """Drop the last -tokens_to_remove positions (a positive value is the length to keep)."""
        keep = tokens_to_remove if tokens_to_remove > 0 else self.length + tokens_to_remove
        keep = max(0, min(self.length, keep))
        if self.cpu_k is not None:
            self.cpu_k = _slice_cpu(self.cpu_k, keep)
            self.cpu_v = _slice_cpu(self.cpu_v, keep)
        self.length = keep

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        self._select_batch(beam_idx)

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        self._select_batch(indices)

    def batch_repeat_interleave(self, repeats: int) -> None:
        if self.shape is None:
            return
        idx = torch.arange(self.shape[0]).repeat_interleave(repeats)
        self._select_batch(idx)

    # ------------------------------------------------------------------ compressed storage
    def append(self, key_compressor, val_compressor, k: torch.Tensor, v: torch.Tensor) -> tuple[dict, dict]:
        """Compress k, v [B, Hkv, S, D], append them, and return dicts covering every cached position."""
        ck, cv, _, _ = self.append_prepare(key_compressor, val_compressor, k, v)
        return ck, cv

    def append_prepare(self, key_compressor, val_compressor, k: torch.Tensor, v: torch.Tensor,
                       q: torch.Tensor | None = None):
        """append(), and on the GPU also the new queries q [B, Hq, S, D] prepared for scoring
        (key_compressor.prepare_queries): (keys, values, q_rot, q_proj), the last two None on the
        CPU or without q.  On the GPU the new rows are compressed straight into the capacity
        planes and the queries prepared in the same launch (tq_cache_append)."""
        B, H, S, D = k.shape
        if self.shape is not None and self.length > 0 and self.shape != (B, H, D):
            raise ValueError(f"cache holds [B, Hkv, D] = {self.shape}, got {(B, H, D)}")
        codec = {"key_bits": key_compressor.bits, "value_bits": val_compressor.bits,
                 "key_seed": getattr(key_compressor, "seed", None),
                 "value_seed": getattr(val_compressor, "seed", None)}
        if self.length > 0 and self.codec:
            # planes written under other seeds (or bits) would be attended with the wrong Pi/S
            stale = {k: (self.codec.get(k), v) for k, v in codec.items()
                     if self.codec.get(k) is not None and v is not None and self.codec.get(k) != v}
            if stale:
                raise ValueError(f"cache layer holds {self.length} positions compressed with other "
                                 f"settings (cached, new): {stale}")
        self.shape = (B, H, D)
        self.codec = codec
        if k.device.type != "cuda":
            return (*self._append_cpu(key_compressor, val_compressor, k, v), None, None)
        from turboquant_pytorch._ops import ops

        tk, tv, need = self._gpu_room(key_compressor, val_compressor, k)
        q_rot, q_proj = ops().cache_append(
            k, v, q, tk.pi_split, tk.seff_split, tk.cent32, tk.bounds32, key_compressor.mse_bits, tv.pi_split,
            tv.bounds32, val_compressor.bits, tk.s_eff16, self.kp["packed_key_indices"], self.kp["packed_qjl_signs"],
            self.kp["residual_norm"], self.kp["vec_norms"], self.vp["packed_indices"], self.vp["vec_norms"],
            self.length)
        self.length = need
        ck, cv = self.strided()
        return (ck, cv, q_rot, q_proj) if q is not None else (ck, cv, None, None)

    def _gpu_room(self, key_compressor, val_compressor, k: torch.Tensor):
        """Device tables of both compressors, and capacity planes that hold S more rows (grown,
        or re-laid out for other shapes or bit widths); returns (tk, tv, length after the append)."""
        from turboquant_pytorch.compressors import _tables

        B, H, S, D = k.shape
        need = self.length + S
        widths = (_cols(D, key_compressor.mse_bits), _cols(D, 1), _cols(D, val_compressor.bits))
        if self.kp is None or need > self.capacity or self.kp["vec_norms"].shape[:2] != (B, H) or \
                self._widths() != widths:
            self._grow(need, B, H, widths, k.device)
        tk = _tables(key_compressor, k.device, with_qjl=True)
        tv = _tables(val_compressor, k.device, with_qjl=False)
        return tk, tv, need

    def append_attend(self, key_compressor, val_compressor, k: torch.Tensor, v: torch.Tensor, q: torch.Tensor,
                      attention_mask: torch.Tensor | None = None, causal: bool = False, scale: float | None = None,
                      out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """GPU: append_prepare() followed by attention over every cached position
        (turboquant_pytorch.fused.attention_from_prepared), in one operator call
        (tq::cache_attend): the same kernels and results, without the second operator's host
        cost, which bounds a one-token decode step.  Returns the attention output [B, S_q, Hq, D]."""
        if k.device.type != "cuda":
            raise ValueError("append_attend runs on the GPU; use append_prepare on the CPU")
        B, H, S, D = k.shape
        if self.shape is not None and self.length > 0 and self.shape != (B, H, D):
            raise ValueError(f"cache holds [B, Hkv, D] = {self.shape}, got {(B, H, D)}")
        codec = {"key_bits": key_compressor.bits, "value_bits": val_compressor.bits,
                 "key_seed": getattr(key_compressor, "seed", None),
                 "value_seed": getattr(val_compressor, "seed", None)}
        if self.length > 0 and self.codec and codec != self.codec:
            stale = {k_: (self.codec.get(k_), v_) for k_, v_ in codec.items()
                     if self.codec.get(k_) is not None and v_ is not None and self.codec.get(k_) != v_}
            if stale:
                raise ValueError(f"cache layer holds {self.length} positions compressed with other "
                                 f"settings (cached, new): {stale}")
        self.shape = (B, H, D)
        self.codec = codec
        from turboquant_pytorch._ops import ops

        tk, tv, need = self._gpu_room(key_compressor, val_compressor, k)
        if out_dtype not in (torch.float32, torch.float16, torch.bfloat16):
            out_dtype = torch.float32
        mask = attention_mask.to(k.device, torch.float32) if attention_mask is not None else None
        out = ops().cache_attend(
            k, v, q, tk.pi_split, tk.seff_split, tk.cent32, tk.bounds32, key_compressor.mse_bits, tv.pi_split,
            tv.bounds32, val_compressor.bits, tk.s_eff16, self.kp["packed_key_indices"], self.kp["packed_qjl_signs"],
            self.kp["residual_norm"], self.kp["vec_norms"], self.vp["packed_indices"], self.vp["vec_norms"],
            self.length, tk.cent16, tv.cent32, tv.pit_split,
            float(math.sqrt(math.pi / 2) / key_compressor.S.shape[0]),
            float(scale if scale is not None else 1.0 / math.sqrt(D)), bool(causal), mask, out_dtype, 1)
        self.length = need
        return out

    def _widths(self) -> tuple | None:
        if self.kp is None:
            return None
        return (self.kp["packed_key_indices"].shape[-1], self.kp["packed_qjl_signs"].shape[-1],
                self.vp["packed_indices"].shape[-1])

    def strided(self) -> tuple[dict, dict]:
        """GPU dicts over the capacity planes: attend the first `length` rows (kv_stride = capacity)."""
        B, H, D = self.shape
        ck = {name: self.kp[name] for name in _KEY_PLANES}
        cv = {name: self.vp[name] for name in _VAL_PLANES}
        for c in (ck, cv):
            c["shape"] = (B, H, self.length, D)
            c["kv_stride"] = self.capacity
        return ck, cv

    def compact(self) -> tuple[dict, dict]:
        """The cached positions in the compressors' own packed format (contiguous copies)."""
        if self.kp is None:
            return self.cpu_k, self.cpu_v
        B, H, D = self.shape
        L, n = self.length, self.shape[0] * self.shape[1] * self.length
        k = {name: self.kp[name][:, :, :L].contiguous() for name in _KEY_PLANES}
        # explicit row widths: an empty cache (L = 0) has nothing for -1 to infer from
        kw, sw = k["packed_key_indices"].shape[-1], k["packed_qjl_signs"].shape[-1]
        vw = self.vp["packed_indices"].shape[-1]
        ck = {"packed_key_indices": k["packed_key_indices"].reshape(n, kw),
              "packed_qjl_signs": k["packed_qjl_signs"].reshape(n, sw),
              "residual_norm": k["residual_norm"], "vec_norms": k["vec_norms"], "shape": (B, H, L, D)}
        cv = {"packed_indices": self.vp["packed_indices"][:, :, :L].contiguous().reshape(n, vw),
              "vec_norms": self.vp["vec_norms"][:, :, :L].contiguous().reshape(n), "shape": (B, H, L, D)}
        return ck, cv

    def restore(self, keys: dict, values: dict, codec: dict) -> None:
        """Replace the layer's contents with compressor-format dicts (packed on the GPU,
        unpacked on the CPU), as `TurboQuantCache.load` reads them."""
        B, H, S, D = keys["shape"]
        self.reset()
        self.kp = self.vp = None
        self.capacity = 0
        self.shape = (B, H, D)
        self.codec = dict(codec)
        packed = "packed_key_indices" in keys
        dev = keys["residual_norm"].device
        if packed != (dev.type == "cuda"):
            raise ValueError("packed planes are restored onto a GPU device, unpacked dicts onto the CPU")
        if not packed:
            self.cpu_k, self.cpu_v = keys, values
            self.length = S
            return
        self._grow(S, B, H, (keys["packed_key_indices"].shape[-1], keys["packed_qjl_signs"].shape[-1],
                             values["packed_indices"].shape[-1]), dev)
        n = B * H * S
        for name in _KEY_PLANES:
            src = keys[name]
            self.kp[name][:, :, :S] = src.reshape(B, H, S, src.shape[-1]) if src.dim() == 2 and src.shape[0] == n \
                else src.reshape(B, H, S)
        vi = values["packed_indices"]
        self.vp["packed_indices"][:, :, :S] = vi.reshape(B, H, S, vi.shape[-1])
        self.vp["vec_norms"][:, :, :S] = values["vec_norms"].reshape(B, H, S)
        self.length = S

    def _grow(self, need: int, B: int, H: int, widths: tuple, dev) -> None:
        """Capacity planes for at least `need` positions (row widths: key codes, signs, value
        codes), keeping the cached rows."""
        cap = max(need, 2 * self.capacity, _ROUND)
        cap = (cap + _ROUND - 1) // _ROUND * _ROUND
        kw, sw, vw = widths
        kp = {
            "packed_key_indices": torch.zeros(B, H, cap, kw, dtype=torch.uint8, device=dev),
            "packed_qjl_signs": torch.zeros(B, H, cap, sw, dtype=torch.uint8, device=dev),
            "residual_norm": torch.zeros(B, H, cap, dtype=torch.float16, device=dev),
            "vec_norms": torch.zeros(B, H, cap, dtype=torch.float16, device=dev),
        }
        vp = {
            "packed_indices": torch.zeros(B, H, cap, vw, dtype=torch.uint8, device=dev),
            "vec_norms": torch.zeros(B, H, cap, dtype=torch.float16, device=dev),
        }
        if self.kp is not None and self.length > 0:
            L = self.length
            for name in _KEY_PLANES:
                kp[name][:, :, :L] = self.kp[name][:, :, :L]
            for name in _VAL_PLANES:
                vp[name][:, :, :L] = self.vp[name][:, :, :L]
        self.kp, self.vp, self.capacity = kp, vp, cap

    def _append_cpu(self, key_compressor, val_compressor, k, v) -> tuple[dict, dict]:
        ck = key_compressor.compress(k)
        cv = val_compressor.compress(v)
        if self.cpu_k is None or self.length == 0:
            self.cpu_k, self.cpu_v = ck, cv
        else:
            self.cpu_k = _cat_cpu(self.cpu_k, ck)
            self.cpu_v = _cat_cpu(self.cpu_v, cv)
        self.length = self.cpu_k["shape"][2]
        return self.cpu_k, self.cpu_v

    def _select_batch(self, idx: torch.Tensor) -> None:
        if self.length == 0 or self.shape is None:
            return
        if self.kp is not None:
            i = idx.to(self.kp["vec_norms"].device)
            self.kp = {name: t.index_select(0, i) for name, t in self.kp.items()}
            self.vp = {name: t.index_select(0, i) for name, t in self.vp.items()}
            self.shape = (int(i.numel()),) + self.shape[1:]
        else:
            self.cpu_k = _select_cpu(self.cpu_k, idx)
            self.cpu_v = _select_cpu(self.cpu_v, idx)
            self.shape = (int(idx.numel()),) + self.shape[1:]


def _cols(d: int, b: int) -> int:
    """Bytes of a packed row of d b-bit codes (bit_ops.py:162-164)."""
    return (d * b + 7) // 8


def _cat_cpu(a: dict, b: dict) -> dict:
    """Concatenate two unpacked CPU dicts of one layer along the sequence."""
    B, H, S1, D = a["shape"]
    S2 = b["shape"][2]
    out = {"shape": (B, H, S1 + S2, D)}
    for name, t in a.items():
        if name == "shape":
            continue
        u = b[name]
        if t.dim() >= 3:  # [B, H, S, ...]
            out[name] = torch.cat([t, u], dim=2)
        else:  # flat rows [B*H*S, ...] (value indices / norms)
            t4 = t.reshape(B, H, S1, *t.shape[1:])
            u4 = u.reshape(B, H, S2, *u.shape[1:])
            out[name] = torch.cat([t4, u4], dim=2).reshape(B * H * (S1 + S2), *t.shape[1:])
    return out


def _slice_cpu(a: dict, keep: int) -> dict:
    B, H, S, D = a["shape"]
    out = {"shape": (B, H, keep, D)}
    for name, t in a.items():
        if name == "shape":
            continue
        if t.dim() >= 3:
            out[name] = t[:, :, :keep].contiguous()
        else:
            out[name] = t.reshape(B, H, S, *t.shape[1:])[:, :, :keep].reshape(B * H * keep, *t.shape[1:])
    return out


def _select_cpu(a: dict, idx: torch.Tensor) -> dict:
    B, H, S, D = a["shape"]
    idx = idx.to("cpu")
    out = {"shape": (int(idx.numel()), H, S, D)}
    for name, t in a.items():
        if name == "shape":
            continue
        if t.dim() >= 3:
            out[name] = t.index_select(0, idx)
        else:
            t4 = t.reshape(B, H, S, *t.shape[1:]).index_select(0, idx)
            out[name] = t4.reshape(-1, *t.shape[1:])
    return out


class TurboQuantCache(Cache):
    """A transformers ``Cache`` whose layers hold TurboQuant-compressed keys and values."""

    def __init__(self, **kwargs):
        super().__init__(layer_class_to_replicate=TurboQuantCacheLayer)

    def layer(self, layer_idx: int) -> TurboQuantCacheLayer:
        while len(self.layers) <= layer_idx:
            self.layers.append(TurboQuantCacheLayer())
        return self.layers[layer_idx]

    def append(self, layer_idx: int, key_compressor, val_compressor, k: torch.Tensor,
               v: torch.Tensor) -> tuple[dict, dict]:
        """Compress and append one layer's new keys/values; return dicts over all cached positions."""
        if layer_idx is None:
            raise ValueError("TurboQuantCache needs attention modules with a layer_idx")
        return self.layer(layer_idx).append(key_compressor, val_compressor, k, v)

    def append_attend(self, layer_idx: int, key_compressor, val_compressor, k: torch.Tensor, v: torch.Tensor,
                      q: torch.Tensor, attention_mask: torch.Tensor | None = None, causal: bool = False,
                      scale: float | None = None, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
        """append_prepare() and the attention over every cached position in one operator call
        on the GPU (see TurboQuantCacheLayer.append_attend)."""
        if layer_idx is None:
            raise ValueError("TurboQuantCache needs attention modules with a layer_idx")
        return self.layer(layer_idx).append_attend(key_compressor, val_compressor, k, v, q, attention_mask, causal,
                                                   scale, out_dtype)

    def append_prepare(self, layer_idx: int, key_compressor, val_compressor, k: torch.Tensor, v: torch.Tensor,
                       q: torch.Tensor | None = None):
        """append() plus the new queries prepared in the same launch on the GPU:
        (keys, values, q_rot, q_proj) (see TurboQuantCacheLayer.append_prepare)."""
        if layer_idx is None:
            raise ValueError("TurboQuantCache needs attention modules with a layer_idx")
        return self.layer(layer_idx).append_prepare(key_compressor, val_compressor, k, v, q)

    def save(self, path, metadata: dict | None = None) -> None:
        """Write every non-empty layer's cached positions to `path` (format turboquant-kv, one
        group per layer named ``layer<i>``, with the compressors' bits and seeds)."""
        from turboquant_pytorch.serialize import save_groups

        groups = []
        for i, lay in enumerate(self.layers):
            if lay.length == 0 or lay.shape is None:
                continue
            keys, values = lay.compact()
            groups.append({"name": f"layer{i}", "keys": keys, "values": values, **lay.codec})
        save_groups(path, groups, metadata)

    @classmethod
    def load(cls, path, device="cpu") -> "TurboQuantCache":
        """A cache holding what `save` wrote; packed planes go to a GPU `device`, unpacked
        dicts to the CPU.  Decoding continues with compressors of the recorded bits and seeds."""
        from turboquant_pytorch.serialize import FormatError, load_groups

        groups, _ = load_groups(path, device)
        cache = cls()
        for g in groups:
            name = g["name"]
            if not (name.startswith("layer") and name[5:].isdigit()):
                raise FormatError(f"cache groups are named layer<i>, found {name!r}")
            if g["keys"] is None or g["values"] is None:
                raise FormatError(f"{name}: a cache layer needs keys and values")
            codec = {k: g[k] for k in ("key_bits", "value_bits", "key_seed", "value_seed")}
            cache.layer(int(name[5:])).restore(g["keys"], g["values"], codec)
        return cache

    def nbytes(self) -> int:
        """Bytes of compressed planes currently cached (positions in use only)."""
        total = 0
        for lay in self.layers:
            if lay.length == 0 or lay.shape is None:
                continue
            B, H, D = lay.shape
            if lay.kp is not None:
                per_pos = sum(t[0, 0, 0].numel() * t.element_size() for t in lay.kp.values())
                per_pos += sum(t[0, 0, 0].numel() * t.element_size() for t in lay.vp.values())
                total += per_pos * B * H * lay.length
            else:
                for c in (lay.cpu_k, lay.cpu_v):
                    total += sum(t.numel() * t.element_size() for n, t in c.items() if n != "shape")
        return total
