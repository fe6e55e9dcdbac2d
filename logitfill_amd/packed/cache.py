"""Packed history cache plus the model-dtype residual page, on the device.

Drop-in for the reference's ``logitfill.packed.cache`` (``src/logitfill/packed/cache.py``):
``PackedKVManager``, ``LogitFillCache`` and the per-layer ``_LayerStore`` keep
the same names, constructor arguments, methods and attributes (``table``,
``hist_k``, ``hist_v``, ``hist_len``, ``tail_k``, ``tail_v``, ``length``,
``append``, ``dequantize``, ``commit``, ``layer_length``, ``reset``, ``seq_len``).

Storage differs from the reference, which re-concatenates the whole history on
every flush (``cache.py:64-81``): each layer owns capacity-strided device arrays
in the reference byte layout -- ``k_code[t] [B, n_kv, cap, words_t]``,
``k_scale/k_min[t] [B, n_kv, width_t, cap/k_group]``, ``k_value16``, ``v_code``,
``v_scale``, ``v_min`` -- and the page-compress kernel writes each full page in
place.  ``hist_k``/``hist_v`` return views of sequence 0's slice, shaped
exactly as the reference's tensors.  Capacity doubles when exceeded.

Extension: ``batch_size`` sequences per manager (the reference raises for
batch != 1, ``cache.py:136-137``); ``commit`` then takes ``[batch, n_kv, T, D]``.
"""
from __future__ import annotations

import os
from typing import Optional

import torch

from logitfill_amd import _native
from logitfill_amd.packed.layout import (
    _ptr,
    device_tables,
    make_layer_struct,
    sm_page_elems,
    tier_tables,
    tier_widths,
    value_words,
)


def _check_device(device) -> torch.device:
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError(
            f"logitfill_amd keeps the packed cache on a ROCm device; got {device} (there is no CPU path)")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


class _LayerStore:
    """One layer's packed history and residual page for ``batch`` sequences (reference ``cache.py:16-90``)."""

    def __init__(self, levels, page_size: int, k_group_size: int, v_group_size: int, bit_v: int, *,
                 device="cuda", batch: int = 1, capacity_tokens: int = 0):
        self.device = _check_device(device)
        levels = torch.as_tensor(levels, dtype=torch.int64).to(self.device)
        built = tier_tables(levels)
        self.table = built["tiers"]
        self.table["tier"] = built["tier"]
        self.page_size = int(page_size)
        self.k_group_size = int(k_group_size)
        self.v_group_size = int(v_group_size)
        self.bit_v = int(bit_v)
        if self.page_size % self.k_group_size:
            raise ValueError(f"page_size {page_size} is not a multiple of k_group_size {k_group_size}")
        self.n_kv, self.head_dim = (int(x) for x in levels.shape)
        if self.bit_v < 16 and self.head_dim % self.v_group_size:
            raise ValueError(f"head dim {self.head_dim} is not divisible by value group {v_group_size}")
        if self.bit_v < 16 and self.bit_v not in (2, 4, 8):
            raise ValueError(f"bit_v must be 2, 4, 8 or >= 16, got {bit_v}")
        self.batch = int(batch)
        self.widths, self.words = tier_widths(self.table)
        self._tables_dev = device_tables(self.table, self.device)
        self._cap = 0
        self._s: dict | None = None
        self._struct = None
        self.hist_lens = [0] * self.batch
        self.tail_lens = [0] * self.batch
        self._tail_k: Optional[torch.Tensor] = None
        self._tail_v: Optional[torch.Tensor] = None
        self._tail_len_dev: Optional[torch.Tensor] = None
        self._tail_dirty = True
        self.decode_plan = None        # cached work plan, owned by the decode dispatcher
        # Deferred flushes (extension): full residual pages (b, dst_page) not yet packed.  Set
        # by the manager; every reader of the history packs them first.
        self.defer_flush = False
        self._pending: list[tuple[int, int]] = []
        if capacity_tokens:
            self.reserve(capacity_tokens)

    # ---- reference attributes (sequence 0) ---------------------------------
    @property
    def hist_len(self) -> int:
        return self.hist_lens[0]

    @property
    def tail_len(self) -> int:
        return self.tail_lens[0]

    @property
    def length(self) -> int:
        return self.hist_len + self.tail_len

    def lengths(self) -> list[int]:
        return [h + t for h, t in zip(self.hist_lens, self.tail_lens)]

    @property
    def tail_k(self) -> Optional[torch.Tensor]:
        return None if self.tail_lens[0] == 0 else self._tail_k[0, :, : self.tail_lens[0]]

    @property
    def tail_v(self) -> Optional[torch.Tensor]:
        return None if self.tail_lens[0] == 0 else self._tail_v[0, :, : self.tail_lens[0]]

    @property
    def hist_k(self) -> Optional[dict]:
        return self.history_views(0)[0]

    @property
    def hist_v(self) -> Optional[dict]:
        return self.history_views(0)[1]

    def history_views(self, b: int = 0):
        """Reference-shaped views of sequence ``b``'s packed history (``cache.py:64-81``), or ``(None, None)``."""
        self.flush()
        H = self.hist_lens[b]
        if H == 0:
            return None, None
        s = self._s
        G = H // self.k_group_size
        hist_k = {t: {"code": s["k_code"][t][b, :, :H], "scale": s["k_scale"][t][b, :, :, :G],
                      "min": s["k_min"][t][b, :, :, :G]} for t in range(3)}
        hist_k[3] = {"value": s["k_value16"][b, :, :H]}
        if self.bit_v >= 16:
            hist_v = {"value": s["v_value16"][b, :, :H]}
        else:
            hist_v = {"code": s["v_code"][b, :, :H], "scale": s["v_scale"][b, :, :H], "min": s["v_min"][b, :, :H]}
        return hist_k, hist_v

    def page_scale_copy(self, b: int = 0):
        """Sequence ``b``'s pages of the page-major Key scale/min copy (``[n_kv, pages,
        16 * blocks]`` fp16, the matrix-core decode kernel's form of the Key scales and mins), or
        None when the layer keeps none or holds no page."""
        self.flush()
        if self._s is None or "k_sm_page" not in self._s or self.hist_lens[b] == 0:
            return None
        return self._s["k_sm_page"][b, :, : self.hist_lens[b] // self.page_size]

    def export_reference(self, b: int = 0):
        """Contiguous copies of ``history_views(b)``: the exact tensors the reference would hold."""
        hk, hv = self.history_views(b)
        if hk is None:
            return None, None
        return ({t: {k: v.contiguous() for k, v in d.items()} for t, d in hk.items()},
                {k: v.contiguous() for k, v in hv.items()})

    # ---- storage -------------------------------------------------------------
    def reserve(self, tokens: int) -> None:
        """Grow the capacity to at least ``tokens`` history tokens (doubling, page aligned)."""
        P = self.page_size
        need = -(-int(tokens) // P) * P
        if need <= self._cap:
            return
        cap = max(need, 2 * self._cap)
        old, old_cap = self._s, self._cap
        B, H, D, dev = self.batch, self.n_kv, self.head_dim, self.device
        W, WD = self.widths, self.words
        groups = cap // self.k_group_size
        s = {
            "k_code": [torch.zeros(B, H, cap, WD[t], dtype=torch.int32, device=dev) for t in range(3)],
            "k_scale": [torch.ones(B, H, W[t], groups, dtype=torch.float16, device=dev) for t in range(3)],
            "k_min": [torch.zeros(B, H, W[t], groups, dtype=torch.float16, device=dev) for t in range(3)],
            "k_value16": torch.zeros(B, H, cap, W[3], dtype=torch.float16, device=dev),
        }
        if self.k_group_size == P and sum(WD):
            # page-major copy of the Key scales / mins for the matrix-core decode kernel (the
            # packers write it beside the reference arrays; lf_common.hpp: sm_page)
            s["k_sm_page"] = torch.zeros(B, H, groups, sm_page_elems(WD), dtype=torch.float16, device=dev)
        if self.bit_v >= 16:
            s["v_value16"] = torch.zeros(B, H, cap, D, dtype=torch.float16, device=dev)
        else:
            vg = D // self.v_group_size
            s["v_code"] = torch.zeros(B, H, cap, value_words(D, self.bit_v), dtype=torch.int32, device=dev)
            s["v_scale"] = torch.zeros(B, H, cap, vg, dtype=torch.float16, device=dev)
            s["v_min"] = torch.zeros(B, H, cap, vg, dtype=torch.float16, device=dev)
        if old is not None and old_cap:
            og = old["k_scale"][0].shape[-1]
            for t in range(3):
                s["k_code"][t][:, :, :old_cap].copy_(old["k_code"][t])
                s["k_scale"][t][..., :og].copy_(old["k_scale"][t])
                s["k_min"][t][..., :og].copy_(old["k_min"][t])
            for name in ("k_value16", "v_value16", "v_code", "v_scale", "v_min"):
                if name in s:
                    s[name][:, :, :old_cap].copy_(old[name])
            if "k_sm_page" in s:
                s["k_sm_page"][:, :, :og].copy_(old["k_sm_page"])
        self._s, self._cap = s, cap
        self._struct = None

    @property
    def capacity(self) -> int:
        return self._cap

    def layer_struct(self) -> _native.PackedLayer:
        """The ``lf_packed_layer`` describing this store (rebuilt after a reallocation)."""
        if self._s is None:
            self.reserve(self.page_size)
        if self._struct is None:
            s = self._s
            self._struct = make_layer_struct(
                self.table, self._tables_dev, batch=self.batch, n_kv=self.n_kv, head_dim=self.head_dim,
                cap_tokens=self._cap, cap_kgroups=int(s["k_scale"][0].shape[-1]), page_size=self.page_size,
                k_group=self.k_group_size, v_group=self.v_group_size, bit_v=self.bit_v,
                k_code=s["k_code"], k_scale=s["k_scale"], k_min=s["k_min"], k_value16=s["k_value16"],
                v_code=s.get("v_code"), v_scale=s.get("v_scale"), v_min=s.get("v_min"),
                v_value16=s.get("v_value16"), k_sm_page=s.get("k_sm_page"))
        return self._struct

    def tail_buffers(self):
        """``(tail_k, tail_v)`` ``[B, n_kv, page_size, D]`` in the model dtype (None before the first append)."""
        return self._tail_k, self._tail_v

    def tail_len_device(self) -> torch.Tensor:
        """int32 ``[B]`` residual lengths on the device, re-uploaded (asynchronously, from pinned
        memory, on the current stream) after they change."""
        if self._tail_dirty or self._tail_len_dev is None:
            self._tail_len_dev = _native.upload(self.tail_lens, torch.int32, self.device)
            self._tail_dirty = False
        return self._tail_len_dev

    # ---- reference behaviour -------------------------------------------------
    def reset(self) -> None:
        """``cache.py:41-46``: forget history and tail (storage is kept for reuse)."""
        self.hist_lens = [0] * self.batch
        self.tail_lens = [0] * self.batch
        self._tail_dirty = True
        self.decode_plan = None
        self._pending = []

    def append(self, key: torch.Tensor, value: torch.Tensor) -> None:
        """``cache.py:48-62`` for one sequence: ``key/value [n_kv, T, D]``; flushes full pages."""
        if self.batch != 1:
            raise ValueError("append takes one sequence; use append_batch for batched stores")
        if key.shape[0] != value.shape[0] or key.shape[1] != value.shape[1]:
            raise ValueError("Key and Value pages do not match")
        self.append_batch(key.unsqueeze(0), value.unsqueeze(0))

    def append_batch(self, key: torch.Tensor, value: torch.Tensor, lengths=None) -> None:
        """Append tokens to every sequence: ``key/value [B, n_kv, T, D]``.

        Sequence b appends ``key[b, :, :lengths[b]]`` (all ``T`` tokens when
        ``lengths`` is None).  Fills each residual page; every page that fills
        is packed in place by the page-compress kernel (``cache.py:54-62`` then
        ``_flush`` :64-81).
        """
        shape = key.shape
        # one token for every sequence into residual pages that stay below full: the decode
        # step's commit, checked and enqueued with as little host work as possible
        if (lengths is None and len(shape) == 4 and shape[2] == 1 and shape == value.shape
                and shape[0] == self.batch and shape[1] == self.n_kv and shape[3] == self.head_dim
                and self._tail_k is not None and not self._pending and max(self.tail_lens) + 1 < self.page_size
                and key.dtype == value.dtype and key.is_cuda and value.is_cuda
                and key.is_contiguous() and value.is_contiguous()):
            self._append_one(key, value)
            return
        if key.shape != value.shape:
            raise ValueError("Key and Value pages do not match")
        B, H, T, D = (int(x) for x in key.shape)
        if B != self.batch or H != self.n_kv or D != self.head_dim:
            raise ValueError(f"expected [{self.batch}, {self.n_kv}, T, {self.head_dim}], got {tuple(key.shape)}")
        if not key.is_cuda or not value.is_cuda:
            raise RuntimeError("logitfill_amd keeps the packed cache on a ROCm device (there is no CPU path)")
        P = self.page_size
        lens = [T] * B if lengths is None else [int(x) for x in lengths]
        if len(lens) != B or min(lens) < 0 or max(lens) > T:
            raise ValueError("lengths must give 0 <= length <= T for every sequence")
        if max(lens) == 0:
            return
        self.flush()
        if self._tail_k is None:
            self._tail_k = torch.zeros(B, H, P, D, dtype=key.dtype, device=self.device)
            self._tail_v = torch.zeros(B, H, P, D, dtype=value.dtype, device=self.device)
        if key.dtype != self._tail_k.dtype:
            key = key.to(self._tail_k.dtype)
        if value.dtype != self._tail_v.dtype:
            value = value.to(self._tail_v.dtype)
        key = key.detach()
        value = value.detach()

        tail_jobs, src_jobs, rest = [], [], {}
        fill: dict[tuple[int, int], list[int]] = {}
        hist_pages = [h // P for h in self.hist_lens]
        new_tail = list(self.tail_lens)
        for b in range(B):
            Tb = lens[b]
            if Tb == 0:
                continue
            tl = self.tail_lens[b]
            n1 = min(Tb, P - tl)
            fill.setdefault((tl, n1), []).append(b)
            pos = n1
            if tl + n1 == P:
                tail_jobs.append((b, 0, hist_pages[b]))
                hist_pages[b] += 1
                new_tail[b] = 0
            else:
                new_tail[b] = tl + n1
            while Tb - pos >= P:
                src_jobs.append((b, pos, hist_pages[b]))
                hist_pages[b] += 1
                pos += P
            if pos < Tb:
                rest[b] = (pos, Tb)
                new_tail[b] = Tb - pos
        # 1) complete the residual pages
        for (tl, n1), bs in fill.items():
            if len(bs) == B:
                self._tail_k[:, :, tl:tl + n1].copy_(key[:, :, :n1])
                self._tail_v[:, :, tl:tl + n1].copy_(value[:, :, :n1])
            else:
                idx = _native.upload(bs, torch.int64, self.device)
                self._tail_k[idx, :, tl:tl + n1] = key[idx, :, :n1]
                self._tail_v[idx, :, tl:tl + n1] = value[idx, :, :n1]
        # 2) pack full pages in place -- or, for a deferring store on a step that only completes
        # residual pages, leave them full in the residual buffers until flush()
        defer = self.defer_flush and bool(tail_jobs) and not src_jobs and not rest
        if tail_jobs or src_jobs:
            self.reserve(max(hist_pages) * P)
            if defer:
                for b, _, page in tail_jobs:
                    self._pending.append((b, page))
                    hist_pages[b] -= 1
                    new_tail[b] = P
            else:
                if tail_jobs:
                    self._pack(self._tail_k, self._tail_v, tail_jobs)
                if src_jobs:
                    self._pack(key, value, src_jobs)
        # 3) start the next residual pages
        for b, (pos, end) in rest.items():
            n = end - pos
            self._tail_k[b, :, :n].copy_(key[b, :, pos:end])
            self._tail_v[b, :, :n].copy_(value[b, :, pos:end])
        self.hist_lens = [p * P for p in hist_pages]
        self.tail_lens = new_tail
        self._tail_dirty = True

    def _append_one(self, key: torch.Tensor, value: torch.Tensor) -> None:
        """One token per sequence into residual pages that stay below full: ``lf_append_token``
        writes the rows at the device-side lengths and advances them, so nothing is uploaded;
        the host copy of the lengths advances in step."""
        tail_len = self.tail_len_device()
        tk, tv = self._tail_k, self._tail_v
        # the arguments fixed while the tail buffers and the new rows' dtype stay, kept per layer
        key_static = (tk.data_ptr(), tv.data_ptr(), tail_len.data_ptr(), key.dtype)
        cached = self.__dict__.get("_lf_append_static")
        if cached is None or cached[0] != key_static:
            cached = (key_static, (tk.data_ptr(), tv.data_ptr(), _native.dtype_code(tk.dtype), int(tk.shape[2]),
                                   tail_len.data_ptr()), _native.dtype_code(key.dtype))
            self.__dict__["_lf_append_static"] = cached
        _, (ptk, ptv, tdt, cap, ptl), ndt = cached
        st = _native.load().lf_append_token(ptk, ptv, tdt, cap, ptl, key.data_ptr(), value.data_ptr(), ndt,
                                            self.batch, self.n_kv, self.head_dim,
                                            _native.current_stream_ptr(self.device))
        _native.check(st, "lf_append_token")
        self.tail_lens = [t + 1 for t in self.tail_lens]

    @property
    def pending(self) -> list[tuple[int, int]]:
        """Deferred page flushes ``(b, dst_page)``."""
        return list(self._pending)

    def flush(self) -> None:
        """Pack the deferred residual pages of this layer (one launch)."""
        if not self._pending:
            return
        jobs = [(b, 0, page) for b, page in self._pending]
        self._pack(self._tail_k, self._tail_v, jobs)
        self._complete_pending()

    def _complete_pending(self) -> None:
        P = self.page_size
        for b, _ in self._pending:
            self.hist_lens[b] += P
            self.tail_lens[b] = 0
        self._pending = []
        self._tail_dirty = True

    def _pack(self, k_src: torch.Tensor, v_src: torch.Tensor, jobs: list) -> None:
        if k_src.stride(-1) != 1:
            k_src = k_src.contiguous()
        if v_src.stride(-1) != 1:
            v_src = v_src.contiguous()
        if k_src.stride() != v_src.stride():
            k_src, v_src = k_src.contiguous(), v_src.contiguous()
        jobs_dev = _native.upload([v for job in jobs for v in job], torch.int32, self.device)
        st = _native.load().lf_pack_pages(
            self.layer_struct(), k_src.data_ptr(), v_src.data_ptr(), _native.dtype_code(k_src.dtype),
            k_src.stride(0), k_src.stride(1), k_src.stride(2), jobs_dev.data_ptr(), len(jobs),
            _native.current_stream_ptr(self.device))
        _native.check(st, "lf_pack_pages")
        self._jobs_keepalive = jobs_dev

    def fill_pages(self, key: torch.Tensor, value: torch.Tensor, pages) -> None:
        """Bulk prefill: pack ``pages[b]`` full pages of ``key/value [B, n_kv, T, D]`` as sequence b's history.

        Sequence b's history must be empty.  Used to build large synthetic caches
        with one launch per layer.
        """
        P = self.page_size
        jobs = []
        for b, n in enumerate(pages):
            if self.hist_lens[b] or self.tail_lens[b]:
                raise ValueError("fill_pages needs an empty sequence")
            jobs.extend((b, p * P, p) for p in range(int(n)))
        if not jobs:
            return
        self.reserve(max(int(n) for n in pages) * P)
        self._pack(key, value, jobs)
        self.hist_lens = [int(n) * P for n in pages]

    def set_tail(self, key: torch.Tensor, value: torch.Tensor, lengths) -> None:
        """Set the residual pages directly: ``key/value [B, n_kv, >=max(lengths), D]``."""
        B, H, _, D = key.shape
        P = self.page_size
        if self._tail_k is None:
            self._tail_k = torch.zeros(B, H, P, D, dtype=key.dtype, device=self.device)
            self._tail_v = torch.zeros(B, H, P, D, dtype=value.dtype, device=self.device)
        for b, n in enumerate(lengths):
            n = int(n)
            if n >= P:
                raise ValueError("a residual page holds fewer than page_size tokens")
            self._tail_k[b, :, :n].copy_(key[b, :, :n])
            self._tail_v[b, :, :n].copy_(value[b, :, :n])
        self.tail_lens = [int(n) for n in lengths]
        self._tail_dirty = True

    def dequantize(self, b: int = 0):
        """``cache.py:83-90``: dense float32 ``(K, V) [n_kv, hist_len, D]`` of sequence ``b`` (HIP kernel)."""
        self.flush()
        H = self.hist_lens[b]
        D = self.head_dim
        k = torch.empty(self.n_kv, H, D, dtype=torch.float32, device=self.device)
        v = torch.empty(self.n_kv, H, D, dtype=torch.float32, device=self.device)
        if H:
            st = _native.load().lf_dequantize(self.layer_struct(), b, H, k.data_ptr(), v.data_ptr(),
                                              _native.current_stream_ptr(self.device))
            _native.check(st, "lf_dequantize")
        return k, v


class PackedKVManager:
    """Per-layer packed KV for ``batch_size`` sequences (reference ``cache.py:93-140``)."""

    def __init__(self, levels, n_q: int, n_kv: int, head_dim: int, page_size: int, k_group_size: int,
                 v_group_size: int, bit_v: int, device, *, batch_size: int = 1, capacity_tokens: int = 0,
                 defer_flush: bool = False):
        self.n_q = int(n_q)
        self.n_kv = int(n_kv)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        self.k_group_size = int(k_group_size)
        self.v_group_size = int(v_group_size)
        self.bit_v = int(bit_v)
        self.device = _check_device(device)
        self.batch_size = int(batch_size)
        if self.n_q % self.n_kv:
            raise ValueError("query heads must divide into KV heads")
        self.seq_len = 0
        self.layers = []
        for level in levels:
            if level is None:
                values = torch.zeros(self.n_kv, head_dim, dtype=torch.int64)
            else:
                values = torch.as_tensor(level, dtype=torch.int64)
            if tuple(values.shape) != (self.n_kv, self.head_dim):
                raise ValueError(f"levels must be [{self.n_kv}, {self.head_dim}] per layer")
            self.layers.append(_LayerStore(values, page_size, k_group_size, v_group_size, bit_v, device=self.device,
                                           batch=self.batch_size, capacity_tokens=capacity_tokens))
        self._workspace: Optional[torch.Tensor] = None
        self._flush_keepalive = None
        self.defer_flush = bool(defer_flush)

    @property
    def defer_flush(self) -> bool:
        """Extension: commits that complete residual pages leave them for ``flush_pending``.

        The reference packs each layer's full page inside that layer's commit
        (``cache.py:54-62``).  Every layer of a decode step fills its page on the
        same token and the packed page is read only by the next step, so a
        deferring manager packs all layers' pages in one launch at the end of the
        step.  Readers of a layer's history (attention, dequantize, the history
        views, the next append) pack that layer's pending pages first.
        """
        return self._defer_flush

    @defer_flush.setter
    def defer_flush(self, value: bool) -> None:
        self._defer_flush = bool(value)
        for layer in self.layers:
            layer.defer_flush = self._defer_flush
            if not value:
                layer.flush()

    def flush_pending(self) -> None:
        """Pack every layer's deferred pages: one ``lf_pack_pages_multi`` launch."""
        todo = [layer for layer in self.layers if layer._pending]
        if not todo:
            return
        if len(todo) == 1:
            todo[0].flush()
            return
        dtypes = {layer._tail_k.dtype for layer in todo}
        n = len(todo)
        structs = (_native.PackedLayer * n)(*[layer.layer_struct() for layer in todo])
        srcs = (_native.PackSource * n)()
        for i, layer in enumerate(todo):
            tk, tv = layer._tail_k, layer._tail_v
            srcs[i] = _native.PackSource(tk.data_ptr(), tv.data_ptr(), tk.stride(0), tk.stride(1), tk.stride(2))
        st = _native.LF_E_UNSUPPORTED if len(dtypes) != 1 else None
        if st is None:
            dev_structs = _native.upload(bytes(structs), torch.uint8, self.device)
            dev_srcs = _native.upload(bytes(srcs), torch.uint8, self.device)
            jobs = [(i, b, 0, page) for i, layer in enumerate(todo) for b, page in layer._pending]
            jobs_dev = _native.upload([v for job in jobs for v in job], torch.int32, self.device)
            st = _native.load().lf_pack_pages_multi(
                dev_structs.data_ptr(), structs, dev_srcs.data_ptr(), srcs, n, _native.dtype_code(dtypes.pop()),
                jobs_dev.data_ptr(), len(jobs), _native.current_stream_ptr(self.device))
            self._flush_keepalive = (dev_structs, dev_srcs, jobs_dev)
        if st == _native.LF_E_UNSUPPORTED:
            # shapes outside the multi-layer kernel: one pack launch per layer
            for layer in todo:
                layer.flush()
            return
        _native.check(st, "lf_pack_pages_multi")
        for layer in todo:
            layer._complete_pending()

    def reset(self) -> None:
        self.seq_len = 0
        for layer in self.layers:
            layer.reset()

    def layer_length(self, layer_idx: int) -> int:
        return self.layers[layer_idx].length

    def commit(self, layer_idx: int, key: torch.Tensor, value: torch.Tensor, lengths=None) -> None:
        """Append ``key/value [batch, n_kv, T, D]`` to layer ``layer_idx`` (reference ``cache.py:135-140``).

        ``lengths`` (extension): per-sequence token counts for ragged batches.
        """
        if key.shape[0] != self.batch_size:
            raise NotImplementedError(
                f"this manager holds {self.batch_size} sequence(s); got a batch of {key.shape[0]}")
        if key.requires_grad or value.requires_grad:
            key, value = key.detach(), value.detach()
        self.layers[layer_idx].append_batch(key, value, lengths)
        if layer_idx == len(self.layers) - 1:
            self.seq_len = self.layers[layer_idx].length

    def workspace(self, nbytes: int) -> torch.Tensor:
        """Shared decode workspace: split-K partials (grown on demand, needs no clearing)."""
        if self._workspace is None or self._workspace.numel() < nbytes:
            self._workspace = torch.empty(int(nbytes), dtype=torch.uint8, device=self.device)
        return self._workspace


try:
    from transformers.cache_utils import Cache as _HFCache
except ImportError:  # pragma: no cover - transformers is optional for the cache itself
    _HFCache = object


def _init_hf_base(obj) -> None:
    """Run the transformers ``Cache`` constructor with no cache layers.  transformers 5.x
    requires ``layers`` (or a layer class); 4.x takes no arguments; without transformers the
    base is ``object``."""
    if _HFCache is object:
        return
    import inspect

    params = inspect.signature(_HFCache.__init__).parameters
    if "layers" in params:
        _HFCache.__init__(obj, layers=[])
    else:
        _HFCache.__init__(obj)


class LogitFillCache(_HFCache):
    """transformers ``Cache`` view of a ``PackedKVManager`` (reference ``cache.py:149-183``).

    Passed as ``past_key_values`` so that a model's forward and ``generate`` derive positions
    and mask sizes from the packed sequence length.  It holds no tensors: the packed attention
    forward reads and commits the manager itself, so ``update`` is an error, and beam search
    (``reorder_cache``) is not supported.  Works with transformers 4.x (``get_mask_sizes``
    receives the cache positions) and 5.x (it receives the query length).
    """

    def __init__(self, manager: PackedKVManager):
        _init_hf_base(self)
        self.manager = manager

    # -- lengths ------------------------------------------------------------------------------
    def get_seq_length(self, layer_idx: int = 0) -> int:
        return int(self.manager.seq_len)

    def get_query_offset(self, layer_idx: int = 0) -> int:
        return int(self.manager.seq_len)

    def get_mask_sizes(self, query, layer_idx: int = 0):
        """``(kv_length, kv_offset)``: the packed tokens plus the ``query`` tokens (an int, or
        the tensor of cache positions older transformers pass), offset 0."""
        q_len = int(query) if isinstance(query, int) else int(query.shape[0])
        return int(self.manager.seq_len) + q_len, 0

    def get_max_length(self, layer_idx: int | None = None) -> int:
        return -1  # grows without a bound

    def get_max_cache_shape(self, layer_idx: int = 0):
        return None

    @property
    def is_compileable(self) -> bool:
        return False

    # -- writes ---------------------------------------------------------------------------------
    def update(self, key_states, value_states, layer_idx, *args, **kwargs):
        raise RuntimeError("the packed attention forward commits to the PackedKVManager itself; "
                           "LogitFillCache.update must not be reached")

    def note_layer(self, layer_idx: int, seq_len: int) -> None:
        """Called by the attention forward after each layer's commit; the length lives in the
        manager, so there is nothing to record."""

    def reset(self) -> None:
        self.manager.reset()

    def crop(self, tokens_to_remove: int) -> None:
        raise NotImplementedError("packed pages cannot be cropped")

    def reorder_cache(self, beam_idx) -> None:
        raise NotImplementedError("beam search is not supported by the packed cache")


def env_int(name: str, default: int) -> int:
    value = os.environ.get(name)
    return int(value) if value else default
