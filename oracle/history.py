"""Numpy restatement of the per-layer packed store.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Reference: ``src/logitfill/packed/cache.py:16-90`` (``_LayerStore``).  One
sequence, one layer: the BF16 tail grows by ``append``; every full page is
packed and concatenated onto the history -- codes and float16 values along
tokens (axis 1), Key scale/min along groups (axis 2), Value scale/min along
tokens (axis 1).
"""
from __future__ import annotations

import numpy as np

from oracle import layout


class LayerHistory:
    def __init__(self, levels, page_size: int, k_group_size: int, v_group_size: int, bit_v: int):
        self.page_size = int(page_size)
        self.k_group_size = int(k_group_size)
        self.v_group_size = int(v_group_size)
        self.bit_v = int(bit_v)
        self.table = layout.layer_table(np.asarray(levels))
        self.hist_k = None
        self.hist_v = None
        self.hist_len = 0
        self.tail_k = None          # float32 [heads, tail, dim] (exact model-dtype values)
        self.tail_v = None

    @property
    def tail_len(self) -> int:
        return 0 if self.tail_k is None else int(self.tail_k.shape[1])

    @property
    def length(self) -> int:
        return self.hist_len + self.tail_len

    def append(self, key: np.ndarray, value: np.ndarray) -> None:
        """``cache.py:48-62``: concatenate onto the tail, flush every full page."""
        key = np.asarray(key, dtype=np.float32)
        value = np.asarray(value, dtype=np.float32)
        if key.shape[0] != value.shape[0] or key.shape[1] != value.shape[1]:
            raise ValueError("Key and Value pages do not match")
        self.tail_k = key if self.tail_k is None else np.concatenate((self.tail_k, key), axis=1)
        self.tail_v = value if self.tail_v is None else np.concatenate((self.tail_v, value), axis=1)
        while self.tail_len >= self.page_size:
            page_k = self.tail_k[:, : self.page_size]
            page_v = self.tail_v[:, : self.page_size]
            self.tail_k = self.tail_k[:, self.page_size:]
            self.tail_v = self.tail_v[:, self.page_size:]
            if self.tail_k.shape[1] == 0:
                self.tail_k = None
                self.tail_v = None
            self._flush(page_k, page_v)

    def _flush(self, key: np.ndarray, value: np.ndarray) -> None:
        """``cache.py:64-81``: pack the page and concatenate along the reference axes."""
        packed_k = layout.quantize_key_page(key, self.table, self.k_group_size)
        packed_v = layout.quantize_value_page(value, self.bit_v, self.v_group_size)
        if self.hist_k is None:
            self.hist_k = packed_k
            self.hist_v = packed_v
        else:
            for code in (0, 1, 2):
                hk, pk = self.hist_k[code], packed_k[code]
                hk["code"] = np.concatenate((hk["code"], pk["code"]), axis=1)
                hk["scale"] = np.concatenate((hk["scale"], pk["scale"]), axis=2)
                hk["min"] = np.concatenate((hk["min"], pk["min"]), axis=2)
            self.hist_k[3]["value"] = np.concatenate((self.hist_k[3]["value"], packed_k[3]["value"]), axis=1)
            if self.bit_v >= 16:
                self.hist_v["value"] = np.concatenate((self.hist_v["value"], packed_v["value"]), axis=1)
            else:
                for name in ("code", "scale", "min"):
                    self.hist_v[name] = np.concatenate((self.hist_v[name], packed_v[name]), axis=1)
        self.hist_len += int(key.shape[1])

    def dequantize(self):
        """``cache.py:83-90``: dense float32 Key and Value history."""
        heads, dim = self.table["tier"].shape
        if self.hist_k is None:
            empty = np.zeros((heads, 0, dim), dtype=np.float32)
            return empty, empty
        key = layout.dequantize_key(self.hist_len, self.table, self.hist_k, self.k_group_size)
        value = layout.dequantize_value(self.hist_v, self.hist_len, dim, self.bit_v, self.v_group_size)
        return key, value


def pack_history(levels, key: np.ndarray, value: np.ndarray, page_size: int = 128,
                 k_group_size: int = 128, v_group_size: int = 128, bit_v: int = 2) -> LayerHistory:
    """Append ``key/value [heads, T, dim]`` in one call (prefill-style commit)."""
    store = LayerHistory(levels, page_size, k_group_size, v_group_size, bit_v)
    store.append(key, value)
    return store
