"""KV-cache footprint of the packed layout: the reference's analytical count and the bytes
the layout really stores.

``runtime_footprint`` restates the reference's accounting
(``src/logitfill/allocators/memory.py:14-98``): Key payload at each channel's level, Value
payload, per-head packing padding (each head's tier padded to whole 32-bit words), scale/min
per quantised channel and group, one int16 channel index per Key channel, the BF16 residual.

The stored layout pads differently: every head's tier row is as wide as the widest head's
(``width_t = max_h count_t[h]``, reference ``packed/layout.py:57,82``), and the padding
slots keep a scale and a min too.  ``stored_footprint`` counts those bytes -- the ones a
decode step actually reads (it agrees with ``bench.algorithmic_bytes``) -- and
``stored_bytes`` sums the tensors of a live cache layer; the analytical figure understates
both whenever heads differ in their tier counts.  Beside the reference layout a layer stores a
page-major copy of the Key scales and mins (``page_copy_bytes``, the form the matrix-core decode
kernel reads in place of the reference's scale/min arrays: per page and kv head, 8-slot blocks
of the integer tiers, 32 bytes each).
"""
from __future__ import annotations

import numpy as np

from logitfill_amd.packed.layout import sm_page_elems

LEVEL_BITS = np.array([2, 4, 8, 16], dtype=np.int64)


def _check(levels, page_size, k_group_size, v_group_size):
    values = np.asarray(levels, dtype=np.int64)
    if values.ndim != 3:
        raise ValueError(f"levels must be [layers, kv_heads, head_dim], got {values.shape}")
    if np.any((values < 0) | (values > 3)):
        raise ValueError("levels must be in {0, 1, 2, 3}")
    if page_size < 1 or k_group_size < 1 or v_group_size < 1:
        raise ValueError("page and group sizes must be positive")
    if page_size % k_group_size:
        raise ValueError("page_size must be a multiple of k_group_size")
    if values.shape[2] % v_group_size:
        raise ValueError(f"head_dim {values.shape[2]} is not divisible by v_group_size {v_group_size}")
    return values


def _summary(seq_len, hist, residual, values, bit_v, parts, elements):
    total = sum(parts.values())
    bit_k = float(LEVEL_BITS[values].mean()) if values.size else float("nan")
    out = {"seq_len": float(seq_len), "history_tokens": float(hist), "residual_tokens": float(residual),
           "actual_bit_k": bit_k, "bit_v": float(bit_v), "actual_bit_kv": 0.5 * (bit_k + float(bit_v))}
    out.update({name: float(v) for name, v in parts.items()})
    out["total_bytes"] = float(total)
    out["bytes_per_token"] = float(total) / seq_len if seq_len else float("nan")
    out["effective_bit"] = float(total) * 8.0 / elements if elements else float("nan")
    return out


def runtime_footprint(levels, seq_len: int, *, page_size: int = 128, k_group_size: int = 128,
                      v_group_size: int = 128, bit_v: int = 2, dtype_bytes: int = 2) -> dict:
    """Bytes and effective bits of one sequence at ``seq_len`` tokens, counted as the
    reference counts them (per-head word padding; metadata for quantised channels only)."""
    values = _check(levels, page_size, k_group_size, v_group_size)
    L, H, D = values.shape
    hist = int(seq_len) // page_size * page_size
    residual = int(seq_len) - hist
    groups = hist // k_group_size
    channels = L * H * D
    k_payload = hist * int(LEVEL_BITS[values].sum()) / 8.0
    if bit_v >= 16:
        v_payload, v_meta = hist * 16 * channels / 8.0, 0.0
    else:
        v_payload = hist * bit_v * channels / 8.0
        v_meta = float(hist * L * H * (D // v_group_size) * 2 * dtype_bytes)
    k_meta = float((values < 3).sum() * groups * 2 * dtype_bytes)
    index = float(values.size * 2)
    pad = 0
    for bits, code in ((2, 0), (4, 1), (8, 2)):
        per = 32 // bits
        counts = (values == code).sum(axis=-1).reshape(-1)
        pad += int(sum(-(-int(c) // per) * per - int(c) for c in counts if c > 0))
    parts = {"k_payload_bytes": k_payload, "v_payload_bytes": v_payload, "packing_padding_bytes": pad * hist / 8.0,
             "metadata_bytes": k_meta + v_meta + index, "residual_bytes": float(residual * channels * 2 * dtype_bytes)}
    return _summary(seq_len, hist, residual, values, bit_v, parts, float(seq_len * channels * 2))


def stored_footprint(levels, seq_len: int, *, page_size: int = 128, k_group_size: int = 128,
                     v_group_size: int = 128, bit_v: int = 2, dtype_bytes: int = 2) -> dict:
    """Bytes one sequence at ``seq_len`` tokens occupies in the stored layout: per layer and
    kv head, ``words_t = ceil(width_t / (32 / bits_t))`` Key words per token for each integer
    tier and ``width_16`` fp16 values, with ``width_t`` the widest head's count; a scale and a
    min (fp16) per tier slot ``< width_t`` and Key group; Value codes, scale and min; the
    int32 tier tables; the residual in ``dtype_bytes``."""
    values = _check(levels, page_size, k_group_size, v_group_size)
    L, H, D = values.shape
    hist = int(seq_len) // page_size * page_size
    residual = int(seq_len) - hist
    groups = hist // k_group_size
    k_payload = k_meta = tables = page_copy = 0
    for layer in range(L):
        counts = [(values[layer] == code).sum(axis=-1) for code in range(4)]
        widths = [int(c.max()) if c.size else 0 for c in counts]
        words = []
        for t, bits in enumerate((2, 4, 8)):
            per = 32 // bits
            words.append(-(-widths[t] // per))
            k_payload += hist * H * 4 * words[t]
            k_meta += H * widths[t] * groups * 2 * 2
        if k_group_size == page_size and sum(words):
            page_copy += (hist // page_size) * H * 2 * sm_page_elems(words)
        k_payload += hist * H * widths[3] * 2
        # index [H, width] + count [H] + local [H, D] (int32) per tier, and the [H, D] tier map
        tables += sum(4 * (H * w + H + H * D) for w in widths) + 4 * H * D
    channels = L * H * D
    if bit_v >= 16:
        v_payload, v_meta = hist * channels * 2, 0
    else:
        v_payload = hist * L * H * (D * bit_v // 32) * 4
        v_meta = hist * L * H * (D // v_group_size) * 2 * 2
    parts = {"k_payload_bytes": float(k_payload), "v_payload_bytes": float(v_payload),
             "metadata_bytes": float(k_meta + v_meta + tables),
             "residual_bytes": float(residual * channels * 2 * dtype_bytes),
             "page_copy_bytes": float(page_copy)}
    out = _summary(seq_len, hist, residual, values, bit_v, parts, float(seq_len * channels * 2))
    out["scale_min_bytes"] = float(k_meta + v_meta)
    out["table_bytes"] = float(tables)
    return out


def stored_bytes(layer, b: int = 0) -> dict:
    """Bytes of sequence ``b`` in a live cache layer (``PackedKVManager.layers[i]``), read off
    its tensors: the packed history rows ``[0, hist_len)`` (``history_views``) and the
    residual tail (the per-layer tier tables are not per sequence and are left out)."""
    hist, tail = int(layer.hist_lens[b]), int(layer.tail_lens[b])
    out = {"k_payload_bytes": 0, "v_payload_bytes": 0, "scale_min_bytes": 0, "residual_bytes": 0,
           "page_copy_bytes": 0}
    hist_k, hist_v = layer.history_views(b)
    if hist_k is not None:
        for t in range(3):
            out["k_payload_bytes"] += hist_k[t]["code"].numel() * hist_k[t]["code"].element_size()
            out["scale_min_bytes"] += sum(hist_k[t][k].numel() * hist_k[t][k].element_size() for k in ("scale", "min"))
        out["k_payload_bytes"] += hist_k[3]["value"].numel() * hist_k[3]["value"].element_size()
        if "value" in hist_v:
            out["v_payload_bytes"] += hist_v["value"].numel() * hist_v["value"].element_size()
        else:
            out["v_payload_bytes"] += hist_v["code"].numel() * hist_v["code"].element_size()
            out["scale_min_bytes"] += sum(hist_v[k].numel() * hist_v[k].element_size() for k in ("scale", "min"))
        copy = layer.page_scale_copy(b)
        if copy is not None:
            out["page_copy_bytes"] = copy.numel() * copy.element_size()
    tk, tv = layer.tail_buffers()
    if tail and tk is not None:
        out["residual_bytes"] = tail * layer.n_kv * layer.head_dim * (tk.element_size() + tv.element_size())
    out["history_tokens"] = hist
    out["residual_tokens"] = tail
    out["total_bytes"] = sum(out[k] for k in ("k_payload_bytes", "v_payload_bytes", "scale_min_bytes", "residual_bytes",
                                              "page_copy_bytes"))
    return out
