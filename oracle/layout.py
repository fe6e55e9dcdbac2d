"""Numpy restatement of the reference byte layout and its numerics.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Every array is numpy.  Floating inputs are float32 arrays holding the exact
values of the model-dtype tensors (a bf16 or fp16 value upcasts to float32
without rounding), so every operation below is the float32 IEEE operation the
reference performs with torch on the CPU:

* ``a / b`` on float32 arrays is correctly rounded IEEE division;
* ``np.rint`` rounds half to even, as ``torch.round`` does;
* ``astype(np.float16)`` rounds to nearest even with overflow to +-inf, as
  ``Tensor.to(torch.float16)`` does.

Reference: ``src/logitfill/packed/layout.py`` (cited per function).
"""
from __future__ import annotations

import numpy as np

LEVEL_BITS = (2, 4, 8, 16)          # level code -> Key bits (layout.py:78, :101)
F32 = np.float32


def asymmetric_codes(grouped: np.ndarray, bits: int):
    """Min-max codes over the last axis.  Reference ``layout.py:12-18``.

    ``grouped`` is float32 ``[..., group]``.  Returns ``(codes int32 [..., group],
    scale float32 [...], low float32 [...])``:

        s    = clamp((max - min) / (2^bits - 1), 1e-5, 1e5)      (float32)
        code = clamp(round_half_even((x - min) / s), 0, 2^bits - 1)
    """
    grouped = np.asarray(grouped, dtype=F32)
    qmax = (1 << int(bits)) - 1
    high = grouped.max(axis=-1, keepdims=True)
    low = grouped.min(axis=-1, keepdims=True)
    scale = np.clip((high - low) / F32(qmax), F32(1e-5), F32(1e5)).astype(F32)
    codes = np.clip(np.rint((grouped - low) / scale), 0, qmax).astype(np.int32)
    return codes, scale[..., 0], low[..., 0]


def pack_ints(codes: np.ndarray, bits: int) -> np.ndarray:
    """LSB-first packing of the last axis into int32 words.  Reference ``layout.py:21-35``.

    Slot ``j`` lands in word ``j // per`` at bit ``(j % per) * bits`` with
    ``per = 32 // bits``; the axis is zero-padded to a multiple of ``per``.
    """
    codes = np.asarray(codes)
    if codes.shape[-1] == 0:
        return np.zeros(codes.shape[:-1] + (0,), dtype=np.int32)
    per = 32 // int(bits)
    pad = (-codes.shape[-1]) % per
    if pad:
        codes = np.concatenate([codes, np.zeros(codes.shape[:-1] + (pad,), codes.dtype)], axis=-1)
    words = codes.shape[-1] // per
    view = codes.reshape(codes.shape[:-1] + (words, per)).astype(np.uint32)
    packed = np.zeros(codes.shape[:-1] + (words,), dtype=np.uint32)
    for slot in range(per):
        packed |= view[..., slot] << np.uint32(slot * bits)
    return packed.view(np.int32)


def unpack_ints(packed: np.ndarray, count: int, bits: int) -> np.ndarray:
    """Inverse of ``pack_ints`` for the first ``count`` slots.  Reference ``layout.py:38-46``."""
    packed = np.asarray(packed)
    if count == 0:
        return np.zeros(packed.shape[:-1] + (0,), dtype=np.int32)
    per = 32 // int(bits)
    slots = np.arange(count)
    words = packed.view(np.uint32)[..., slots // per]
    codes = (words >> ((slots % per) * bits).astype(np.uint32)) & np.uint32((1 << bits) - 1)
    return codes.astype(np.int32)


def tier_tables(levels: np.ndarray) -> dict:
    """Per-tier channel tables.  Reference ``layout.py:49-68``.

    ``levels`` is ``[heads, dim]`` with codes 0=int2, 1=int4, 2=int8, 3=fp16.
    For tier ``t``: ``index[h, :count[h]]`` lists the channels of level ``t`` in
    ascending order (zero padded to ``width = max_h count[h]``), ``local[h, c]``
    is the rank of channel ``c`` inside its tier (-1 elsewhere).  Returns the
    reference's structure ``{"tiers": {t: {...}}, "tier": levels(int32)}``.
    """
    levels = np.asarray(levels)
    heads, dim = levels.shape
    tables = {}
    for code in (0, 1, 2, 3):
        rows = [np.nonzero(levels[h] == code)[0] for h in range(heads)]
        width = max((len(r) for r in rows), default=0)
        index = np.zeros((heads, width), dtype=np.int32)
        count = np.zeros((heads,), dtype=np.int32)
        local = np.full((heads, dim), -1, dtype=np.int32)
        for h, row in enumerate(rows):
            count[h] = len(row)
            if len(row):
                index[h, : len(row)] = row
                local[h, row] = np.arange(len(row), dtype=np.int32)
        tables[code] = {"index": index, "count": count, "local": local, "width": int(width)}
    return {"tiers": tables, "tier": levels.astype(np.int32)}


def layer_table(levels: np.ndarray) -> dict:
    """The table a layer store keeps: tiers 0..3 plus ``"tier"`` (reference ``cache.py:22-24``)."""
    built = tier_tables(levels)
    table = dict(built["tiers"])
    table["tier"] = built["tier"]
    return table


def quantize_key_page(page: np.ndarray, table: dict, group_size: int) -> dict:
    """Pack one Key page ``[heads, tokens, dim]``.  Reference ``layout.py:71-112``.

    Tiers 0..2: per head, the tier's channels are grouped along tokens
    (``group_size`` tokens per group), quantised with ``asymmetric_codes`` and
    packed token-major: ``code [heads, tokens, words]``,
    ``scale/min [heads, width, groups]`` in float16.  Unused slots keep
    scale 1, min 0 and code 0.  Tier 3 stores float16 copies,
    ``value [heads, tokens, width]``.
    """
    page = np.asarray(page, dtype=F32)
    heads, tokens, _dim = page.shape
    if tokens % group_size != 0:
        raise ValueError(f"Key page length {tokens} is not a multiple of {group_size}")
    groups = tokens // group_size
    out = {}
    for code, bits in ((0, 2), (1, 4), (2, 8)):
        index = table[code]["index"]
        count = table[code]["count"]
        width = int(table[code]["width"])
        per = 32 // bits
        words = (width + per - 1) // per if width else 0
        code_out = np.zeros((heads, tokens, words), dtype=np.int32)
        scale = np.ones((heads, width, groups), dtype=np.float16)
        minimum = np.zeros((heads, width, groups), dtype=np.float16)
        for head in range(heads):
            used = int(count[head])
            if used == 0:
                continue
            channels = index[head, :used].astype(np.int64)
            gathered = page[head][:, channels].T                      # [used, tokens]
            grouped = gathered.reshape(used, groups, group_size)
            codes, sc, low = asymmetric_codes(grouped, bits)
            flat = codes.reshape(used, tokens).T                      # [tokens, used]
            padded = np.zeros((tokens, width), dtype=np.int32)
            padded[:, :used] = flat
            code_out[head] = pack_ints(padded, bits)
            scale[head, :used] = sc.astype(np.float16)
            minimum[head, :used] = low.astype(np.float16)
        out[code] = {"code": code_out, "scale": scale, "min": minimum}
    index = table[3]["index"]
    count = table[3]["count"]
    width = int(table[3]["width"])
    values = np.zeros((heads, tokens, width), dtype=np.float16)
    for head in range(heads):
        used = int(count[head])
        if used:
            values[head, :, :used] = page[head][:, index[head, :used].astype(np.int64)].astype(np.float16)
    out[3] = {"value": values}
    return out


def quantize_value_page(page: np.ndarray, bits: int, group_size: int) -> dict:
    """Per-token Value packing.  Reference ``layout.py:115-129``.

    Groups of ``group_size`` consecutive channels per token; codes packed along
    channels: ``code [heads, tokens, dim*bits/32]``, ``scale/min [heads, tokens,
    dim/group_size]`` float16.  ``bits >= 16`` stores float16 copies.
    """
    page = np.asarray(page, dtype=F32)
    heads, tokens, dim = page.shape
    if bits >= 16:
        return {"value": page.astype(np.float16)}
    if dim % group_size != 0:
        raise ValueError(f"head dim {dim} is not divisible by value group {group_size}")
    grouped = page.reshape(heads, tokens, dim // group_size, group_size)
    codes, scale, low = asymmetric_codes(grouped, bits)
    flat = codes.reshape(heads, tokens, dim)
    return {
        "code": pack_ints(flat, bits),
        "scale": scale.astype(np.float16),
        "min": low.astype(np.float16),
    }


def dequantize_key(tokens: int, table: dict, packed: dict, group_size: int) -> np.ndarray:
    """Dense float32 Key history ``[heads, tokens, dim]``.  Reference ``layout.py:132-167``.

    ``restored = code * scale + min`` (two rounded float32 operations), scale
    and min upcast from float16 and broadcast per ``group_size`` tokens; tier 3
    upcasts the stored float16 values.
    """
    tier = table["tier"]
    heads, dim = tier.shape
    out = np.zeros((heads, tokens, dim), dtype=F32)
    if tokens == 0:
        return out
    groups = np.arange(tokens) // group_size
    for code, bits in ((0, 2), (1, 4), (2, 8)):
        index = table[code]["index"]
        count = table[code]["count"]
        block = packed[code]
        for head in range(heads):
            used = int(count[head])
            if used == 0:
                continue
            codes = unpack_ints(block["code"][head, :tokens], used, bits).astype(F32)
            channels = index[head, :used].astype(np.int64)
            scale = block["scale"][head, :used].astype(F32)          # [used, n_groups]
            minimum = block["min"][head, :used].astype(F32)
            restored = codes * scale[:, groups].T + minimum[:, groups].T
            out[head][:, channels] = restored
    index = table[3]["index"]
    count = table[3]["count"]
    for head in range(heads):
        used = int(count[head])
        if used:
            out[head][:, index[head, :used].astype(np.int64)] = packed[3]["value"][head, :tokens, :used].astype(F32)
    return out


def dequantize_value(packed: dict, tokens: int, dim: int, bits: int, group_size: int) -> np.ndarray:
    """Dense float32 Value history ``[heads, tokens, dim]``.  Reference ``layout.py:170-182``."""
    if bits >= 16:
        return packed["value"][:, :tokens].astype(F32)
    heads = packed["code"].shape[0]
    if tokens == 0:
        return np.zeros((heads, 0, dim), dtype=F32)
    codes = unpack_ints(packed["code"][:, :tokens], dim, bits).astype(F32)
    groups = np.arange(dim) // group_size
    scale = packed["scale"][:, :tokens].astype(F32)
    minimum = packed["min"][:, :tokens].astype(F32)
    return (codes * scale[:, :, groups] + minimum[:, :, groups]).reshape(heads, tokens, dim)
