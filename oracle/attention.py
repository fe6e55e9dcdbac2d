"""Numpy restatement of the dense dequantise-then-attend decode path.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``src/logitfill/packed/reference.py:10-56``.  Keys are
``[dequantised history ; tail ; new]`` in float32, values likewise; q head
``i`` reads kv head ``i // (n_q / n_kv)`` (``repeat_kv``); softmax attention
in float32 with ``scale = scaling``; queries aligned to the right edge of the
key sequence when ``q_len > 1``; the result is cast to the query dtype.
"""
from __future__ import annotations

import numpy as np

from oracle import layout


def repeat_kv(states: np.ndarray, repeats: int) -> np.ndarray:
    """``reference.py:10-15``: ``[heads, T, D] -> [heads*repeats, T, D]``, head h feeds h*r..h*r+r-1."""
    if repeats == 1:
        return states
    return np.repeat(states, repeats, axis=0)


def causal_mask(query_len: int, key_len: int):
    """``reference.py:18-27``: right-aligned causal float mask, or None for one query."""
    if query_len == 1:
        return None
    mask = np.zeros((query_len, key_len), dtype=np.float32)
    for index in range(query_len):
        visible = key_len - query_len + index + 1
        if visible < key_len:
            mask[index, visible:] = -np.inf
    return mask


def sdpa(query: np.ndarray, key: np.ndarray, value: np.ndarray, scale: float, mask=None,
         dtype=np.float32) -> np.ndarray:
    """Softmax attention ``[H, Q, D] x [H, T, D] -> [H, Q, D]`` in ``dtype`` arithmetic."""
    q = query.astype(dtype)
    k = key.astype(dtype)
    v = value.astype(dtype)
    scores = np.matmul(q, np.swapaxes(k, -1, -2)) * dtype(scale)
    if mask is not None:
        scores = scores + mask.astype(dtype)
    scores = scores - scores.max(axis=-1, keepdims=True)
    weights = np.exp(scores)
    weights = weights / weights.sum(axis=-1, keepdims=True)
    return np.matmul(weights, v)


def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest even), returned as float32 values."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    rounded = (bits + np.uint64(0x7FFF) + ((bits >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16)
    out = (rounded << np.uint64(16)).astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def round_to_dtype(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bf16":
        return round_to_bf16(x)
    if dtype == "fp16":
        return x.astype(np.float16).astype(np.float32)
    return x.astype(np.float32)


def reference_attention(store, query: np.ndarray, key_new: np.ndarray, value_new: np.ndarray,
                        scaling: float, n_q: int, n_kv: int, out_dtype: str | None = None,
                        dtype=np.float32) -> np.ndarray:
    """``reference.py:30-56`` for one sequence.

    ``store`` is an ``oracle.history.LayerHistory`` (or any object with
    ``dequantize()``, ``tail_k`` and ``tail_v``); ``query [n_q, q_len, D]``,
    ``key_new/value_new [n_kv, q_len, D]`` hold float32 values.  Returns the
    float32 attention output ``[n_q, q_len, D]``, rounded to ``out_dtype``
    ("bf16"/"fp16") when given, as the reference's final cast does.
    """
    key_hist, value_hist = store.dequantize()
    pieces_k = [key_hist]
    pieces_v = [value_hist]
    if store.tail_k is not None and store.tail_k.shape[1] > 0:
        pieces_k.append(np.asarray(store.tail_k, dtype=np.float32))
        pieces_v.append(np.asarray(store.tail_v, dtype=np.float32))
    pieces_k.append(np.asarray(key_new, dtype=np.float32))
    pieces_v.append(np.asarray(value_new, dtype=np.float32))
    key = np.concatenate(pieces_k, axis=1)
    value = np.concatenate(pieces_v, axis=1)
    repeats = n_q // n_kv
    key = repeat_kv(key, repeats)
    value = repeat_kv(value, repeats)
    mask = causal_mask(query.shape[-2], key.shape[-2])
    out = sdpa(np.asarray(query, dtype=np.float32), key, value, scaling, mask, dtype=dtype).astype(np.float32)
    return round_to_dtype(out, out_dtype) if out_dtype else out


class ExportedHistory:
    """A store built from reference-format history tensors (e.g. exported from a device cache)."""

    def __init__(self, levels, hist_k, hist_v, hist_len, tail_k, tail_v, k_group_size, v_group_size, bit_v):
        self.table = layout.layer_table(np.asarray(levels))
        self.hist_k = hist_k
        self.hist_v = hist_v
        self.hist_len = int(hist_len)
        self.tail_k = tail_k
        self.tail_v = tail_v
        self.k_group_size = int(k_group_size)
        self.v_group_size = int(v_group_size)
        self.bit_v = int(bit_v)

    def dequantize(self):
        heads, dim = self.table["tier"].shape
        if self.hist_k is None or self.hist_len == 0:
            empty = np.zeros((heads, 0, dim), dtype=np.float32)
            return empty, empty
        key = layout.dequantize_key(self.hist_len, self.table, self.hist_k, self.k_group_size)
        value = layout.dequantize_value(self.hist_v, self.hist_len, dim, self.bit_v, self.v_group_size)
        return key, value
