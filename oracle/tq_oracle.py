"""CPU oracle for the TurboQuant hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference algorithm (SrzStephen/transformers-turboquant,
src/turboquant_pytorch) used as the checker for the gfx950 kernels.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it;
the product (transformers-turboquant_amd/) never does.

Each function cites the reference lines it restates.  Matrices (Pi, S), the
codebook and boundaries are inputs here: they come from the compressor under
test, whose set-up is pinned separately (tests/test_setup_pins.py).

Floating-point conventions: float32 arithmetic where the reference computes in
float32 (so the decision inputs -- rotated coordinates y and projections -- are
f32 BLAS results comparable to the reference's), float64 for the scoring and
attention estimators so they serve as ground truth for the f32-accumulating
kernels.  Every function is pinned by tests/test_oracle_pins.py, tests/test_setup_pins.py
and the reference vectors under tests/golden/ (known answers, invariants, brute force).
"""

from __future__ import annotations

import math

import numpy as np

# ---------------------------------------------------------------- bit layout


def out_cols(d: int, b: int) -> int:
    """Bytes for d codes of b bits (bit_ops.py:162-164)."""
    return (d * b + 7) // 8


def pack_bits(codes: np.ndarray, b: int) -> np.ndarray:
    """int [N, d] -> uint8 [N, ceil(d*b/8)]; code i at bits [i*b, i*b+b), LSB first,
    each code masked to b bits (bit_ops.py:243-286)."""
    codes = np.asarray(codes, dtype=np.int64) & ((1 << b) - 1)
    n, d = codes.shape
    bits = ((codes[:, :, None] >> np.arange(b)) & 1).astype(np.uint8).reshape(n, d * b)
    nbytes = out_cols(d, b)
    padded = np.zeros((n, nbytes * 8), dtype=np.uint8)
    padded[:, : d * b] = bits
    return np.packbits(padded, axis=1, bitorder="little")


def unpack_bits(packed: np.ndarray, b: int, d: int) -> np.ndarray:
    """uint8 [N, ceil(d*b/8)] -> int32 [N, d] (bit_ops.py:288-326)."""
    packed = np.asarray(packed, dtype=np.uint8)
    bits = np.unpackbits(packed, axis=1, bitorder="little")[:, : d * b].reshape(-1, d, b)
    return (bits.astype(np.int64) << np.arange(b)).sum(-1).astype(np.int32)


# ---------------------------------------------------------------- quantisation


def quantize_searchsorted(y: np.ndarray, boundaries: np.ndarray) -> np.ndarray:
    """code = #{j : boundaries[j] < y}; torch.searchsorted side='left'
    (quantize.py:334-337)."""
    return np.searchsorted(np.asarray(boundaries, np.float32), np.asarray(y, np.float32), side="left").astype(np.int32)


def quantize_argmin(y: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """argmin_j |y - c_j|, first minimum on ties (compressors.py:141-142, :288-289)."""
    diff = np.abs(np.asarray(y, np.float32)[..., None] - np.asarray(centroids, np.float32))
    return diff.argmin(-1).astype(np.int32)


def dequantize(packed: np.ndarray, centroids: np.ndarray, b: int, d: int) -> np.ndarray:
    """f16 centroid lookup of packed codes (quantize.py:341-369)."""
    return np.asarray(centroids, np.float16)[unpack_bits(packed, b, d)]


# ---------------------------------------------------------------- compression


def _rows(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return x.reshape(-1, x.shape[-1])


def rotate(x: np.ndarray, pi: np.ndarray):
    """vn = ||x||, y = (x / (vn + 1e-8)) Pi^T in f32 (compressors.py:104-112)."""
    flat = _rows(x)
    vn = np.sqrt((flat.astype(np.float64) ** 2).sum(-1)).astype(np.float32)
    y = (flat / (vn[:, None] + np.float32(1e-8))) @ np.asarray(pi, np.float32).T
    return flat, vn, y.astype(np.float32)


def key_compress_packed(x, pi, s, centroids, boundaries, mse_bits: int, y=None) -> dict:
    """Packed key compression (compressors.py:99-138).

    If y (the f32 rotated rows) is given it is used for the decisions, so
    codes can be compared bit-exactly against a device that reports its own y.
    Reconstruction uses f16-rounded centroids as at :120-122.
    """
    flat, vn, y_own = rotate(x, pi)
    y = y_own if y is None else np.asarray(y, np.float32).reshape(y_own.shape)
    codes = quantize_searchsorted(y, boundaries)
    c16 = np.asarray(centroids, np.float32).astype(np.float16).astype(np.float32)
    k_mse = (c16[codes] @ np.asarray(pi, np.float32)) * vn[:, None]
    resid = flat - k_mse
    rn = np.sqrt((resid.astype(np.float64) ** 2).sum(-1)).astype(np.float32)
    proj = (resid @ np.asarray(s, np.float32).T).astype(np.float32)
    return {
        "codes": codes,
        "packed_key_indices": pack_bits(codes, mse_bits),
        "proj": proj,
        "packed_qjl_signs": pack_bits((proj >= 0).astype(np.int32), 1),
        "residual_norm": rn.astype(np.float16),
        "vec_norms": vn.astype(np.float16),
        "y": y,
        "k_mse": k_mse,
    }


def key_compress_unpacked(x, pi, s, centroids) -> dict:
    """Unpacked (PyTorch-branch) key compression (compressors.py:139-161)."""
    flat, vn, y = rotate(x, pi)
    idx = quantize_argmin(y, centroids)
    k_mse = (np.asarray(centroids, np.float32)[idx] @ np.asarray(pi, np.float32)) * vn[:, None]
    resid = flat - k_mse
    proj = resid @ np.asarray(s, np.float32).T
    return {
        "k_mse": k_mse.astype(np.float16),
        "qjl_signs": np.where(proj >= 0, 1, -1).astype(np.int8),
        "residual_norm": np.sqrt((resid.astype(np.float64) ** 2).sum(-1)).astype(np.float16),
        "indices": idx,
    }


def value_compress_packed(x, pi, boundaries, bits: int, y=None) -> dict:
    """Packed value compression (compressors.py:271-287)."""
    _, vn, y_own = rotate(x, pi)
    y = y_own if y is None else np.asarray(y, np.float32).reshape(y_own.shape)
    codes = quantize_searchsorted(y, boundaries)
    return {"codes": codes, "packed_indices": pack_bits(codes, bits), "vec_norms": vn.astype(np.float16), "y": y}


def value_compress_unpacked(x, pi, centroids) -> dict:
    """Unpacked value compression (compressors.py:288-294)."""
    _, vn, y = rotate(x, pi)
    return {"indices": quantize_argmin(y, centroids).astype(np.uint8), "vec_norms": vn.astype(np.float16)}


def value_decompress(codes: np.ndarray, vn16: np.ndarray, pi, centroids, dtype=np.float64) -> np.ndarray:
    """(C[codes] Pi) * vn with f32 centroids, in float64 by default (compressors.py:311-317)."""
    c = np.asarray(centroids, dtype)[codes]
    return (c @ np.asarray(pi, dtype)) * np.asarray(vn16, dtype).reshape(-1, 1)


# ---------------------------------------------------------------- scoring


def query_prep(q, pi, s_eff16):
    """q_rot = f16(q Pi^T) (compressors.py:186) and the QJL projection
    q_rot S_eff^T (attention.py:158-167), returned in float64 (unrounded)."""
    qr = (_rows(q).astype(np.float64) @ np.asarray(pi, np.float64).T).astype(np.float32).astype(np.float16)
    qp = qr.astype(np.float64) @ np.asarray(s_eff16, np.float16).astype(np.float64).T
    return qr, qp


def scores_packed(q_rot16, q_proj, codes, sign_bits, rn16, vn16, centroids16, coeff):
    """Asymmetric estimator on packed-format inputs (attention.py:419-461), float64.

    q_rot16 [Nq, d] f16; q_proj [Nq, m]; codes [Nk, d] int; sign_bits [Nk, m] {0,1};
    returns [Nq, Nk] = vn * <q_rot, C[codes]> + coeff * rn * <q_proj, 2*sign - 1>.
    """
    c = np.asarray(centroids16, np.float16).astype(np.float64)[codes]
    t1 = np.asarray(q_rot16, np.float64) @ c.T * np.asarray(vn16, np.float64)[None, :]
    pm = np.asarray(sign_bits, np.float64) * 2.0 - 1.0
    t2 = np.asarray(q_proj, np.float64) @ pm.T * (coeff * np.asarray(rn16, np.float64))[None, :]
    return t1 + t2


def scores_unpacked(q, k_mse16, signs, rn16, s, coeff, dtype=np.float64):
    """PyTorch-branch estimator (compressors.py:201-224), float64 by default."""
    q = _rows(q).astype(dtype)
    t1 = q @ np.asarray(k_mse16, dtype).T
    qs = q @ np.asarray(s, dtype).T
    return t1 + dtype(coeff) * (qs @ np.asarray(signs, dtype).T) * np.asarray(rn16, dtype)[None, :]


def attention(scores, values, scale, mask=None, causal=False, dtype=np.float64):
    """Family forward tail (families/qwen2.py:110-117): softmax(scores*scale + mask) @ values,
    float64 by default.  causal drops keys j > i + Sk - Sq."""
    s = np.asarray(scores, dtype) * dtype(scale)
    if mask is not None:
        s = s + np.asarray(mask, dtype)
    if causal:
        sq, sk = s.shape[-2:]
        i = np.arange(sq)[:, None] + (sk - sq)
        j = np.arange(sk)[None, :]
        s = np.where(j <= i, s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ np.asarray(values, dtype)


# ---------------------------------------------------------------- helpers for tests


def rel_err(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / max(np.linalg.norm(a) * np.linalg.norm(b), 1e-300))


COEFF = lambda m: math.sqrt(math.pi / 2) / m  # noqa: E731  (compressors.py:182)
