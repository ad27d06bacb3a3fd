"""On-disk / wire format for compressed KV planes (format "turboquant-kv", version 1).

The reference keeps compressed keys and values only in memory (its compressor
dicts, compressors.py:114-138, :271-294); this module gives them a versioned,
self-describing container so a compressed cache can be stored, shipped and
restored bit for bit.

Container: safetensors (8-byte little-endian header length, JSON header, raw
little-endian tensor data; read without executing anything from the file).
The header's ``__metadata__`` holds ``format`` = "turboquant-kv", ``version`` =
"1", optional caller metadata under ``user.*`` keys, and ``groups``: a JSON list,
one entry per (keys, values) pair::

    {"name": "layer0", "layout": "packed" | "unpacked", "shape": [B, H, S, D],
     "key_bits": b_k | null, "value_bits": b_v | null,
     "key_seed": s_k | null, "value_seed": s_v | null}

``key_bits`` / ``value_bits`` are the compressors' total bits (keys store
max(b_k - 1, 1)-bit codes plus one QJL sign bit per coordinate); the seeds
name the rotation / QJL matrices (``TurboQuantCompressorV2(D, b_k, seed)``)
needed to decode, when the caller supplies them.  Every plane is stored as
rows in (batch, head, position) order, N = B*H*S rows:

=========================  =========  ===================================
packed layout              dtype      shape
=========================  =========  ===================================
``<name>/k.codes``         uint8      [N, ceil(D * max(b_k-1, 1) / 8)]
``<name>/k.signs``         uint8      [N, ceil(D / 8)]
``<name>/k.rn``            float16    [N]   residual norms
``<name>/k.vn``            float16    [N]   vector norms
``<name>/v.codes``         uint8      [N, ceil(D * b_v / 8)]
``<name>/v.vn``            float16    [N]
=========================  =========  ===================================

Codes and signs are packed LSB first, exactly the bytes of the compressors'
packed dicts.  The unpacked layout stores the reference's PyTorch-branch dicts
(compressors.py:139-161, :288-294): ``k.k_mse`` float16 [N, D], ``k.qjl_signs``
int8 [N, D], ``k.rn`` float16 [N], ``v.indices`` uint8 [N, D], ``v.vn`` float16
[N].  A group may hold keys only or values only.
"""

from __future__ import annotations

import json
import math

import torch
from safetensors.torch import load as _st_load
from safetensors.torch import load_file as _st_load_file
from safetensors.torch import save as _st_save

__all__ = ["FORMAT", "VERSION", "FormatError", "save_compressed", "load_compressed", "dumps", "loads",
           "save_groups", "load_groups", "pack_groups", "unpack_groups"]

FORMAT = "turboquant-kv"
VERSION = 1

# plane name in the file -> (name in the compressor dict, dtype)
_PACKED_K = {"k.codes": ("packed_key_indices", torch.uint8), "k.signs": ("packed_qjl_signs", torch.uint8),
             "k.rn": ("residual_norm", torch.float16), "k.vn": ("vec_norms", torch.float16)}
_PACKED_V = {"v.codes": ("packed_indices", torch.uint8), "v.vn": ("vec_norms", torch.float16)}
_UNPACKED_K = {"k.k_mse": ("k_mse", torch.float16), "k.qjl_signs": ("qjl_signs", torch.int8),
               "k.rn": ("residual_norm", torch.float16)}
_UNPACKED_V = {"v.indices": ("indices", torch.uint8), "v.vn": ("vec_norms", torch.float16)}


class FormatError(ValueError):
    """The data is not a valid turboquant-kv container of a supported version."""


def _layout(keys: dict | None, values: dict | None) -> str:
    kinds = set()
    if keys is not None:
        kinds.add("packed" if "packed_key_indices" in keys else "unpacked")
    if values is not None:
        kinds.add("packed" if "packed_indices" in values else "unpacked")
    if len(kinds) != 1:
        raise ValueError("need keys and/or values, both packed or both unpacked")
    return kinds.pop()


def _cols(layout: str, plane: str, D: int, key_bits, value_bits) -> int | None:
    """Expected trailing dimension of a plane (None: the plane is 1-D)."""
    if plane in ("k.rn", "k.vn", "v.vn"):
        return None
    if layout == "unpacked":
        return D
    if plane == "k.codes":
        return math.ceil(D * max(key_bits - 1, 1) / 8)
    if plane == "k.signs":
        return math.ceil(D / 8)
    return math.ceil(D * value_bits / 8)  # v.codes


def pack_groups(groups: list[dict]) -> tuple[dict[str, torch.Tensor], list[dict]]:
    """Flatten groups {name, keys, values, key_bits, value_bits, key_seed, value_seed} into
    file tensors (contiguous CPU) and the ``groups`` metadata list."""
    tensors: dict[str, torch.Tensor] = {}
    infos = []
    for g in groups:
        name, keys, values = g["name"], g.get("keys"), g.get("values")
        if "/" in name or not name:
            raise ValueError(f"group name {name!r} must be non-empty and contain no '/'")
        layout = _layout(keys, values)
        shape = tuple(int(x) for x in (keys if keys is not None else values)["shape"])
        if keys is not None and values is not None and tuple(values["shape"]) != shape:
            raise ValueError(f"keys shape {shape} != values shape {tuple(values['shape'])}")
        B, H, S, D = shape
        n = B * H * S
        kb, vb = g.get("key_bits"), g.get("value_bits")
        if layout == "packed" and keys is not None and kb is None:
            kb = _infer_bits(keys["packed_key_indices"], n, D, key=True)
        if layout == "packed" and values is not None and vb is None:
            vb = _infer_bits(values["packed_indices"], n, D, key=False)
        info = {"name": name, "layout": layout, "shape": list(shape),
                "key_bits": kb if keys is not None else None, "value_bits": vb if values is not None else None,
                "key_seed": g.get("key_seed") if keys is not None else None,
                "value_seed": g.get("value_seed") if values is not None else None}
        for src, table in ((keys, _PACKED_K if layout == "packed" else _UNPACKED_K),
                           (values, _PACKED_V if layout == "packed" else _UNPACKED_V)):
            if src is None:
                continue
            for plane, (field, dtype) in table.items():
                t = src[field]
                cols = _cols(layout, plane, D, kb, vb)
                want = (n,) if cols is None else (n, cols)
                if t.numel() != math.prod(want) or t.dtype != dtype:
                    raise ValueError(f"{name}: plane {field} has {tuple(t.shape)} {t.dtype}, expected "
                                     f"{want} {dtype}")
                tensors[f"{name}/{plane}"] = t.detach().reshape(want).contiguous().cpu()
        infos.append(info)
    return tensors, infos


def _infer_bits(codes: torch.Tensor, n: int, D: int, key: bool) -> int:
    cols = codes.numel() // max(n, 1)
    for b in range(1, 9):
        code_bits = max(b - 1, 1) if key else b
        if math.ceil(D * code_bits / 8) == cols and (not key or b >= 2):
            return b
    raise ValueError(f"cannot infer bits from {cols} code bytes per row at head_dim {D}")


def unpack_groups(tensors: dict[str, torch.Tensor], infos: list, device="cpu") -> list[dict]:
    """Validate file tensors against the ``groups`` metadata and rebuild compressor dicts."""
    if not isinstance(infos, list):
        raise FormatError("groups metadata must be a list")
    seen = set()
    out = []
    for info in infos:
        try:
            name, layout = str(info["name"]), info["layout"]
            B, H, S, D = (int(x) for x in info["shape"])
            kb, vb = info.get("key_bits"), info.get("value_bits")
        except (KeyError, TypeError, ValueError) as e:
            raise FormatError(f"malformed group entry {info!r}") from e
        if layout not in ("packed", "unpacked") or min(B, H, S, D) < 0:
            raise FormatError(f"group {name}: bad layout {layout!r} or shape")
        n = B * H * S
        g = {"name": name, "key_bits": kb, "value_bits": vb, "key_seed": info.get("key_seed"),
             "value_seed": info.get("value_seed"), "keys": None, "values": None}
        for which, table in (("keys", _PACKED_K if layout == "packed" else _UNPACKED_K),
                             ("values", _PACKED_V if layout == "packed" else _UNPACKED_V)):
            present = [p for p in table if f"{name}/{p}" in tensors]
            if not present:
                continue
            if len(present) != len(table):
                raise FormatError(f"group {name}: {which} planes incomplete ({present})")
            bits = kb if which == "keys" else vb
            if layout == "packed" and not isinstance(bits, int):
                raise FormatError(f"group {name}: packed {which} need integer bits, got {bits!r}")
            d = {"shape": (B, H, S, D)}
            for plane, (field, dtype) in table.items():
                t = tensors[f"{name}/{plane}"]
                seen.add(f"{name}/{plane}")
                cols = _cols(layout, plane, D, kb, vb)
                want = (n,) if cols is None else (n, cols)
                if tuple(t.shape) != want or t.dtype != dtype:
                    raise FormatError(f"group {name}: plane {plane} is {tuple(t.shape)} {t.dtype}, "
                                      f"expected {want} {dtype}")
                d[field] = _to_dict_shape(field, which, layout, t, B, H, S, D).to(device)
            g[which] = d
        if g["keys"] is None and g["values"] is None:
            raise FormatError(f"group {name}: no planes")
        out.append(g)
    extra = set(tensors) - seen
    if extra:
        raise FormatError(f"tensors not described by any group: {sorted(extra)[:4]}")
    return out


def _to_dict_shape(field: str, which: str, layout: str, t: torch.Tensor, B, H, S, D) -> torch.Tensor:
    """File rows -> the shapes the compressors return."""
    if which == "keys":
        if field in ("residual_norm", "vec_norms"):
            return t.reshape(B, H, S)
        if layout == "unpacked":
            return t.reshape(B, H, S, D)
        return t
    return t  # value planes are flat rows in both layouts


def _header(infos: list, metadata: dict | None) -> dict[str, str]:
    meta = {"format": FORMAT, "version": str(VERSION), "groups": json.dumps(infos)}
    for k, v in (metadata or {}).items():
        meta[f"user.{k}"] = str(v)
    return meta


def _check_header(meta: dict | None) -> list:
    if not meta or meta.get("format") != FORMAT:
        raise FormatError(f"not a {FORMAT} container")
    try:
        version = int(meta.get("version", ""))
    except ValueError as e:
        raise FormatError(f"bad version {meta.get('version')!r}") from e
    if version > VERSION or version < 1:
        raise FormatError(f"{FORMAT} version {version} is not supported (this reader handles 1..{VERSION})")
    try:
        return json.loads(meta["groups"])
    except (KeyError, json.JSONDecodeError) as e:
        raise FormatError("missing or malformed groups metadata") from e


def _group_arg(keys, values, key_compressor, value_compressor) -> dict:
    return {"name": "kv", "keys": keys, "values": values,
            "key_bits": getattr(key_compressor, "bits", None), "value_bits": getattr(value_compressor, "bits", None),
            "key_seed": getattr(key_compressor, "seed", None), "value_seed": getattr(value_compressor, "seed", None)}


def save_compressed(path, keys: dict | None = None, values: dict | None = None, key_compressor=None,
                    value_compressor=None, metadata: dict | None = None) -> None:
    """Write one compressed (keys, values) pair; the compressors supply bits and seeds."""
    tensors, infos = pack_groups([_group_arg(keys, values, key_compressor, value_compressor)])
    with open(path, "wb") as f:
        f.write(_container(tensors, _header(infos, metadata)))


def dumps(keys: dict | None = None, values: dict | None = None, key_compressor=None, value_compressor=None,
          metadata: dict | None = None) -> bytes:
    """The bytes `save_compressed` would write."""
    tensors, infos = pack_groups([_group_arg(keys, values, key_compressor, value_compressor)])
    return _container(tensors, _header(infos, metadata))


def _container(tensors: dict[str, torch.Tensor], meta: dict[str, str]) -> bytes:
    """The container's bytes, deterministic for the same planes and metadata: the safetensors
    writer keeps ``__metadata__`` in a hash map, so its key order (and the file's bytes) would
    differ between processes.  The header is re-emitted with ``__metadata__`` first, its keys
    sorted, and the tensor entries in the writer's data order, space-padded to 8 bytes as
    safetensors pads it; the tensor data is unchanged."""
    raw = _st_save(tensors, metadata=meta)  # pack_groups made the tensors contiguous CPU copies
    n = int.from_bytes(raw[:8], "little")
    head = json.loads(raw[8:8 + n])
    entries = sorted(((k, v) for k, v in head.items() if k != "__metadata__"), key=lambda kv: kv[1]["data_offsets"])
    canon = {"__metadata__": dict(sorted(head.get("__metadata__", {}).items()))}
    canon.update(entries)
    text = json.dumps(canon, separators=(",", ":")).encode()
    text += b" " * (-len(text) % 8)
    return len(text).to_bytes(8, "little") + text + raw[8 + n:]


def _read_meta(path) -> dict:
    with open(path, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise FormatError("truncated container")
        n = int.from_bytes(head, "little")
        if n <= 0 or n > 64 << 20:
            raise FormatError("bad header length")
        try:
            return json.loads(f.read(n)).get("__metadata__") or {}
        except (json.JSONDecodeError, UnicodeDecodeError) as e:
            raise FormatError("malformed header") from e


def _meta_from_bytes(data: bytes) -> dict:
    if len(data) < 8:
        raise FormatError("truncated container")
    n = int.from_bytes(data[:8], "little")
    if n <= 0 or 8 + n > len(data):
        raise FormatError("bad header length")
    try:
        return json.loads(data[8:8 + n]).get("__metadata__") or {}
    except (json.JSONDecodeError, UnicodeDecodeError) as e:
        raise FormatError("malformed header") from e


def _single(groups: list[dict], meta: dict) -> tuple[dict | None, dict | None, dict]:
    if len(groups) != 1:
        raise FormatError(f"expected one (keys, values) group, found {len(groups)}")
    g = groups[0]
    info = {k: g[k] for k in ("key_bits", "value_bits", "key_seed", "value_seed")}
    info.update({k[5:]: v for k, v in meta.items() if k.startswith("user.")})
    return g["keys"], g["values"], info


def load_compressed(path, device="cpu") -> tuple[dict | None, dict | None, dict]:
    """Read a pair written by `save_compressed`: (keys, values, info) with compressor-format dicts
    on `device`; info holds bits, seeds and the caller's metadata."""
    meta = _read_meta(path)
    infos = _check_header(meta)
    try:
        tensors = _st_load_file(str(path))
    except Exception as e:  # the safetensors parser rejects corrupt files
        raise FormatError(f"corrupt container: {e}") from e
    return _single(unpack_groups(tensors, infos, device), meta)


def loads(data: bytes, device="cpu") -> tuple[dict | None, dict | None, dict]:
    """`load_compressed` from bytes."""
    meta = _meta_from_bytes(data)
    infos = _check_header(meta)
    try:
        tensors = _st_load(data)
    except Exception as e:
        raise FormatError(f"corrupt container: {e}") from e
    return _single(unpack_groups(tensors, infos, device), meta)


def save_groups(path, groups: list[dict], metadata: dict | None = None) -> None:
    """Write several named (keys, values) groups (see `pack_groups`) into one container."""
    tensors, infos = pack_groups(groups)
    with open(path, "wb") as f:
        f.write(_container(tensors, _header(infos, metadata)))


def load_groups(path, device="cpu") -> tuple[list[dict], dict]:
    """Read every group of a container: (groups as `unpack_groups` returns them, caller metadata)."""
    meta = _read_meta(path)
    infos = _check_header(meta)
    try:
        tensors = _st_load_file(str(path))
    except Exception as e:
        raise FormatError(f"corrupt container: {e}") from e
    return unpack_groups(tensors, infos, device), {k[5:]: v for k, v in meta.items() if k.startswith("user.")}
