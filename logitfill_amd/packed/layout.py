"""Packed byte layout: tier tables (host) and the device page packers / dequantisers.

Same names, arguments and return structures as the reference's
``logitfill.packed.layout`` (``src/logitfill/packed/layout.py``):

* ``asymmetric_codes``, ``pack_ints``, ``unpack_ints`` -- the element-wise
  helpers (``layout.py:12-46``), as HIP kernels;
* ``tier_tables(levels)`` -- host integer work on the tiny ``[heads, dim]``
  level map (``layout.py:49-68``);
* ``quantize_key_page`` / ``quantize_value_page`` -- run the HIP page-compress
  kernel on one page and return the reference dictionaries
  (``layout.py:71-129``);
* ``dequantize_key`` / ``dequantize_value`` -- run the HIP dequantise kernel on
  reference-format tensors (``layout.py:132-182``).

Device functions require ROCm tensors and the built extension; they raise
otherwise (there is no CPU path).
"""
from __future__ import annotations

import torch

from logitfill_amd import _native

LEVEL_BITS = (2, 4, 8, 16)


def tier_tables(levels: torch.Tensor) -> dict:
    """Per-tier channel tables of a ``[heads, dim]`` level map (reference ``layout.py:49-68``).

    For tier ``t``: ``index [heads, width]`` ascending channel ids zero padded
    to ``width = max_h count[h]``; ``count [heads]``; ``local [heads, dim]`` the
    rank of each channel inside its tier (-1 elsewhere).  ``"tier"`` is the
    level map as int32.
    """
    levels = torch.as_tensor(levels)
    if levels.dim() != 2:
        raise ValueError(f"levels must be [heads, dim], got {tuple(levels.shape)}")
    if levels.numel() and (int(levels.min()) < 0 or int(levels.max()) > 3):
        raise ValueError("levels must be in {0, 1, 2, 3}")
    heads, dim = levels.shape
    device = levels.device
    host = levels.detach().to("cpu", torch.int64)
    tables = {}
    for code in (0, 1, 2, 3):
        rows = [torch.nonzero(host[h] == code, as_tuple=False).flatten() for h in range(heads)]
        width = max((int(r.numel()) for r in rows), default=0)
        index = torch.zeros(heads, width, dtype=torch.int32)
        count = torch.zeros(heads, dtype=torch.int32)
        local = torch.full((heads, dim), -1, dtype=torch.int32)
        for h, row in enumerate(rows):
            count[h] = int(row.numel())
            if row.numel():
                index[h, : row.numel()] = row.to(torch.int32)
                local[h, row] = torch.arange(row.numel(), dtype=torch.int32)
        tables[code] = {"index": index.to(device), "count": count.to(device), "local": local.to(device),
                        "width": width}
    return {"tiers": tables, "tier": levels.to(torch.int32)}


def value_words(dim: int, bits: int) -> int:
    """int32 words of one token's packed Value row: ``ceil(dim * bits / 32)``, the last word zero
    padded (``layout.py:27-29``)."""
    per = 32 // int(bits)
    return -(-int(dim) // per)


def tier_widths(table: dict) -> tuple[list[int], list[int]]:
    """``(width_t for t=0..3, words_t for t=0..2)`` of a layer table."""
    widths = [int(table[t]["width"]) for t in range(4)]
    words = [(widths[t] + (16 >> t) - 1) // (16 >> t) for t in range(3)]
    return widths, words


def asymmetric_codes(grouped: torch.Tensor, bits: int):
    """Min-max codes over the last axis on the device (reference ``layout.py:12-18``).

    ``grouped [..., group]`` (bfloat16, float16 or float32; computed in float32, the
    reference's arithmetic on its float32 inputs).  Returns ``(codes int32 [..., group],
    scale float32 [...], low float32 [...])`` with ``scale = clamp((max - min) / (2^bits - 1),
    1e-5, 1e5)`` and ``codes = clamp(round_half_even((x - min) / scale), 0, 2^bits - 1)``.
    """
    device = _require_device(grouped)
    x = grouped.contiguous()
    lead = tuple(x.shape[:-1])
    group = int(x.shape[-1]) if x.dim() else 1
    n_groups = x.numel() // max(group, 1)
    codes = torch.empty(x.shape, dtype=torch.int32, device=device)
    scale = torch.empty(lead, dtype=torch.float32, device=device)
    low = torch.empty(lead, dtype=torch.float32, device=device)
    if n_groups and group:
        st = _native.load().lf_asymmetric_codes(x.data_ptr(), _native.dtype_code(x.dtype), n_groups, group, int(bits),
                                                codes.data_ptr(), scale.data_ptr(), low.data_ptr(),
                                                _native.current_stream_ptr(device))
        _native.check(st, "lf_asymmetric_codes")
    return codes, scale, low


def pack_ints(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first packing of the last axis into int32 words on the device (reference
    ``layout.py:21-35``): slot ``j`` goes to word ``j // per`` at bit ``(j % per) * bits``,
    ``per = 32 // bits``, the last word zero padded.  ``codes`` are non-negative integers."""
    device = _require_device(codes)
    n = int(codes.shape[-1])
    per = 32 // int(bits)
    out = torch.zeros(*codes.shape[:-1], -(-n // per), dtype=torch.int32, device=device)
    rows = codes.numel() // n if n else 0
    if rows:
        src = codes.to(torch.int32).contiguous()
        st = _native.load().lf_pack_ints(src.data_ptr(), rows, n, int(bits), out.data_ptr(),
                                         _native.current_stream_ptr(device))
        _native.check(st, "lf_pack_ints")
    return out


def unpack_ints(packed: torch.Tensor, count: int, bits: int) -> torch.Tensor:
    """The first ``count`` slots of each row of packed int32 words (reference
    ``layout.py:38-46``), on the device; ``[..., words] -> [..., count]`` int32."""
    device = _require_device(packed)
    n_words = int(packed.shape[-1])
    out = torch.zeros(*packed.shape[:-1], int(count), dtype=torch.int32, device=device)
    rows = packed.numel() // n_words if n_words else 0
    if count and rows:
        src = packed.to(torch.int32).contiguous()
        st = _native.load().lf_unpack_ints(src.data_ptr(), rows, n_words, int(count), int(bits), out.data_ptr(),
                                           _native.current_stream_ptr(device))
        _native.check(st, "lf_unpack_ints")
    elif count and not n_words:
        raise IndexError(f"cannot unpack {count} slots from rows of zero words")
    return out


def _require_device(*tensors: torch.Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "logitfill_amd runs on ROCm devices only; got a tensor on "
                f"{t.device} (there is no CPU path)")
        device = t.device
    return device


def _ptr(t) -> int:
    return 0 if t is None or t.numel() == 0 else int(t.data_ptr())


def sm_page_elems(words) -> int:
    """fp16 elements of one page's block of the page-major Key scale/min copy (``k_sm_page``):
    8-slot blocks of the integer tiers in the decode kernel's K-step order -- int2 2 * ceil(w / 4)
    steps, int4 ceil(w / 4), int8 ceil(ceil(w / 2) / 4), 4 blocks a step -- each 8 scales then 8
    mins (``lf_common.hpp``: sm_page)."""
    steps = 2 * -(-int(words[0]) // 4) + -(-int(words[1]) // 4) + -(-(-(-int(words[2]) // 2)) // 4)
    return 16 * 4 * steps


def make_layer_struct(table: dict, table_dev: dict, *, batch: int, n_kv: int, head_dim: int,
                      cap_tokens: int, cap_kgroups: int, page_size: int, k_group: int, v_group: int,
                      bit_v: int, k_code, k_scale, k_min, k_value16, v_code=None, v_scale=None,
                      v_min=None, v_value16=None, k_sm_page=None) -> _native.PackedLayer:
    """Fill an ``lf_packed_layer`` from device tensors (kept alive by the caller)."""
    widths, words = tier_widths(table)
    s = _native.PackedLayer()
    for t in range(3):
        s.k_code[t] = _ptr(k_code[t])
        s.k_scale[t] = _ptr(k_scale[t])
        s.k_min[t] = _ptr(k_min[t])
    s.k_value16 = _ptr(k_value16)
    s.v_code = _ptr(v_code)
    s.v_scale = _ptr(v_scale)
    s.v_min = _ptr(v_min)
    s.v_value16 = _ptr(v_value16)
    s.k_sm_page = _ptr(k_sm_page)
    for t in range(4):
        s.tier_index[t] = _ptr(table_dev[t]["index"])
        s.tier_count[t] = _ptr(table_dev[t]["count"])
        s.k_width[t] = widths[t]
    for t in range(3):
        s.k_words[t] = words[t]
    s.batch, s.n_kv, s.head_dim = batch, n_kv, head_dim
    s.cap_tokens, s.cap_kgroups = cap_tokens, cap_kgroups
    s.page_size, s.k_group, s.v_group, s.bit_v = page_size, k_group, v_group, bit_v
    s.v_words = value_words(head_dim, bit_v) if bit_v < 16 else 0
    s.v_groups = head_dim // v_group if bit_v < 16 else 0
    return s


def device_tables(table: dict, device) -> dict:
    """Contiguous int32 device copies of ``index``/``count`` per tier."""
    return {t: {"index": table[t]["index"].to(device=device, dtype=torch.int32).contiguous(),
                "count": table[t]["count"].to(device=device, dtype=torch.int32).contiguous()}
            for t in range(4)}


def _quantize_page(key: torch.Tensor, value: torch.Tensor, table: dict, k_group: int, v_group: int,
                   bit_v: int) -> tuple[dict, dict]:
    """Pack one page ``key/value [heads, tokens, dim]`` with one kernel launch.

    Returns the reference's ``(packed_k, packed_v)`` dictionaries, as
    ``quantize_key_page`` and ``quantize_value_page`` do for that page.
    """
    device = _require_device(key, value)
    heads, tokens, dim = key.shape
    if tuple(value.shape) != (heads, tokens, dim):
        raise ValueError("Key and Value pages do not match")
    if tokens % k_group != 0:
        raise ValueError(f"Key page length {tokens} is not a multiple of {k_group}")
    if bit_v < 16 and dim % v_group != 0:
        raise ValueError(f"head dim {dim} is not divisible by value group {v_group}")
    widths, words = tier_widths(table)
    tdev = device_tables(table, device)
    groups = tokens // k_group
    k_code = [torch.zeros(heads, tokens, words[t], dtype=torch.int32, device=device) for t in range(3)]
    k_scale = [torch.ones(heads, widths[t], groups, dtype=torch.float16, device=device) for t in range(3)]
    k_min = [torch.zeros(heads, widths[t], groups, dtype=torch.float16, device=device) for t in range(3)]
    k_value16 = torch.zeros(heads, tokens, widths[3], dtype=torch.float16, device=device)
    if bit_v < 16:
        v = {"code": torch.zeros(heads, tokens, value_words(dim, bit_v), dtype=torch.int32, device=device),
             "scale": torch.zeros(heads, tokens, dim // v_group, dtype=torch.float16, device=device),
             "min": torch.zeros(heads, tokens, dim // v_group, dtype=torch.float16, device=device)}
        vv = dict(v_code=v["code"], v_scale=v["scale"], v_min=v["min"])
    else:
        v = {"value": torch.zeros(heads, tokens, dim, dtype=torch.float16, device=device)}
        vv = dict(v_value16=v["value"])
    # A single "page" spanning all tokens keeps the reference's group layout.
    s = make_layer_struct(table, tdev, batch=1, n_kv=heads, head_dim=dim, cap_tokens=tokens,
                          cap_kgroups=groups, page_size=tokens, k_group=k_group, v_group=v_group,
                          bit_v=bit_v, k_code=k_code, k_scale=k_scale, k_min=k_min, k_value16=k_value16, **vv)
    kc = key.contiguous()
    vc = value.contiguous()
    jobs = torch.tensor([[0, 0, 0]], dtype=torch.int32, device=device)
    lib = _native.load()
    st = lib.lf_pack_pages(s, kc.data_ptr(), vc.data_ptr(), _native.dtype_code(kc.dtype),
                           0, kc.stride(0), kc.stride(1), jobs.data_ptr(), 1,
                           _native.current_stream_ptr(device))
    _native.check(st, "lf_pack_pages")
    packed_k = {t: {"code": k_code[t], "scale": k_scale[t], "min": k_min[t]} for t in range(3)}
    packed_k[3] = {"value": k_value16}
    return packed_k, v


def quantize_key_page(page: torch.Tensor, table: dict, group_size: int) -> dict:
    """Pack one Key page ``[heads, tokens, dim]`` on the device (reference ``layout.py:71-112``)."""
    packed_k, _ = _quantize_page(page, page, table, group_size, page.shape[-1], 16)
    return packed_k


def quantize_value_page(page: torch.Tensor, bits: int, group_size: int) -> dict:
    """Per-token Value packing on the device (reference ``layout.py:115-129``)."""
    heads, tokens, dim = page.shape
    if bits >= 16:
        _require_device(page)
        return {"value": page.to(torch.float16)}
    if bits not in (2, 4, 8):
        raise ValueError(f"bit_v must be 2, 4, 8 or >= 16, got {bits}")
    levels = torch.zeros(heads, dim, dtype=torch.int64)
    built = tier_tables(levels)
    table = dict(built["tiers"])
    table["tier"] = built["tier"]
    _, packed_v = _quantize_page(page, page, table, tokens, group_size, bits)
    return packed_v


def _dequantize(tokens: int, table: dict, packed_k, packed_v, k_group: int, v_group: int, bit_v: int,
                dim: int, heads: int, device):
    widths, _ = tier_widths(table)
    tdev = device_tables(table, device)
    empty = torch.empty(0, device=device)
    if packed_k is not None:
        k_code = [packed_k[t]["code"][:, :tokens].contiguous() for t in range(3)]
        k_scale = [packed_k[t]["scale"].contiguous() for t in range(3)]
        k_min = [packed_k[t]["min"].contiguous() for t in range(3)]
        k_value16 = packed_k[3]["value"][:, :tokens].contiguous()
        cap_kgroups = -(-tokens // k_group)
        for t in range(3):
            if widths[t]:
                cap_kgroups = int(k_scale[t].shape[2])
    else:
        k_code = k_scale = k_min = [empty] * 3
        k_value16 = empty
        cap_kgroups = -(-tokens // k_group)
    vv = {}
    if packed_v is not None:
        if bit_v < 16:
            vv = dict(v_code=packed_v["code"][:, :tokens].contiguous(),
                      v_scale=packed_v["scale"][:, :tokens].contiguous(),
                      v_min=packed_v["min"][:, :tokens].contiguous())
        else:
            vv = dict(v_value16=packed_v["value"][:, :tokens].contiguous())
    s = make_layer_struct(table, tdev, batch=1, n_kv=heads, head_dim=dim, cap_tokens=tokens,
                          cap_kgroups=cap_kgroups, page_size=k_group, k_group=k_group, v_group=v_group,
                          bit_v=bit_v, k_code=k_code, k_scale=k_scale, k_min=k_min, k_value16=k_value16, **vv)
    k_out = torch.empty(heads, tokens, dim, dtype=torch.float32, device=device) if packed_k is not None else None
    v_out = torch.empty(heads, tokens, dim, dtype=torch.float32, device=device) if packed_v is not None else None
    if tokens:
        st = _native.load().lf_dequantize(s, 0, tokens, _ptr(k_out), _ptr(v_out), _native.current_stream_ptr(device))
        _native.check(st, "lf_dequantize")
    return k_out, v_out


def dequantize_key(tokens: int, table: dict, packed: dict, group_size: int) -> torch.Tensor:
    """Dense float32 Key history ``[heads, tokens, dim]`` (reference ``layout.py:132-167``)."""
    tier = table["tier"]
    heads, dim = tier.shape
    device = _require_device(packed[0]["code"])
    k, _ = _dequantize(tokens, table, packed, None, group_size, dim, 16, dim, heads, device)
    return k


def dequantize_value(packed: dict, tokens: int, dim: int, bits: int, group_size: int) -> torch.Tensor:
    """Dense float32 Value history ``[heads, tokens, dim]`` (reference ``layout.py:170-182``)."""
    ref = packed["code"] if bits < 16 else packed["value"]
    device = _require_device(ref)
    heads = int(ref.shape[0])
    levels = torch.zeros(heads, dim, dtype=torch.int64)
    built = tier_tables(levels)
    table = dict(built["tiers"])
    table["tier"] = built["tier"]
    _, v = _dequantize(tokens, table, None, packed, group_size, group_size, bits, dim, heads, device)
    return v
