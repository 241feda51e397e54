"""Float64 closed-form attention with explicit per-query loops (NumPy).

    out[i] = sum_j softmax_j(scale * q[i] . k[j] + mask[i, j]) v[j]

This is the mathematical definition behind every attention call on the
reference path (``F.scaled_dot_product_attention`` / ``varlen_attn``), written
independently of torch so that it can pin the torch-based oracle.  Small
cases only.
"""

from __future__ import annotations

import math

import numpy as np


def attention_rows(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    visible: np.ndarray,
    scale: float | None = None,
) -> np.ndarray:
    """One head: ``q`` (Lq, D), ``k``/``v`` (Lk, D), ``visible`` (Lq, Lk) bool.
    A query with no visible key gets zeros (the flash-attention convention)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else scale
    out = np.zeros((q.shape[0], v.shape[1]), dtype=np.float64)
    for i in range(q.shape[0]):
        keys = np.flatnonzero(visible[i])
        if keys.size == 0:
            continue
        scores = np.array([scale * float(np.dot(q[i], k[j])) for j in keys])
        weights = np.exp(scores - scores.max())
        weights /= weights.sum()
        out[i] = (weights[:, None] * v[keys]).sum(axis=0)
    return out


def visible_mask(
    len_q: int, len_k: int, n_keys: int | None = None, causal: str | None = None
) -> np.ndarray:
    """Which keys each query sees: keys ``< n_keys`` and, for ``causal``,
    ``j <= i`` (``"top_left"``, torch's ``is_causal``) or
    ``j <= i + n_keys - len_q`` (``"bottom_right"``, flash varlen
    ``window_size=(-1, 0)``)."""
    n_keys = len_k if n_keys is None else n_keys
    i = np.arange(len_q)[:, None]
    j = np.arange(len_k)[None, :]
    mask = np.broadcast_to(j < n_keys, (len_q, len_k))
    if causal == "top_left":
        mask = mask & (j <= i)
    elif causal == "bottom_right":
        mask = mask & (j <= i + n_keys - len_q)
    elif causal is not None:
        raise ValueError(causal)
    return mask


def attention_bhld(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    n_keys: np.ndarray | None = None,
    causal: str | None = None,
    scale: float | None = None,
) -> np.ndarray:
    """Batched heads: ``q`` (B, Hq, Lq, D), ``k``/``v`` (B, Hkv, Lk, D), query
    head ``h`` reading kv head ``h // (Hq // Hkv)``; ``n_keys`` (B,) caps each
    sequence's keys."""
    batch, heads_q, len_q, _ = q.shape
    heads_kv, len_k = k.shape[1], k.shape[2]
    group = heads_q // heads_kv
    out = np.zeros(q.shape[:3] + (v.shape[-1],), dtype=np.float64)
    for b in range(batch):
        n = len_k if n_keys is None else int(n_keys[b])
        visible = visible_mask(len_q, len_k, n, causal)
        for h in range(heads_q):
            out[b, h] = attention_rows(q[b, h], k[b, h // group], v[b, h // group], visible, scale)
    return out
