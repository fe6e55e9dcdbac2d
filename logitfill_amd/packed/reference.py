"""Decode-attention call for the packed cache.

Drop-in for the reference's ``logitfill.packed.reference``
(``src/logitfill/packed/reference.py``):

* ``packed_attention(manager, layer_idx, query, key_new, value_new, scaling)``
  -- the new query token(s) of each sequence go to the HIP split-K decode
  kernel over the packed pages, the residual page and the new tokens
  (``lf_decode_attention``); this replaces ``_kernel_attention`` and the CUDA
  kernel it launches (``reference.py:59-109``).  Several query tokens (chunked
  scoring, speculative decoding), which the reference sends to its dense path
  (``reference.py:62``), stay on the kernel with the right-aligned causal mask
  (``reference.py:18-27,48``).
* Shapes no kernel serves -- ``bit_v != 2`` -- run ``reference_attention`` on
  the device: HIP dequantisation of the history, then float32 softmax attention
  with the right-aligned causal mask (``reference.py:18-56``).

Nothing here runs on the CPU: a missing extension or a CPU tensor raises.
"""
from __future__ import annotations

import ctypes
import functools
import os
import warnings
from collections import Counter

import numpy as np
import torch

from logitfill_amd import _native
from logitfill_amd.packed.cache import env_int


def repeat_kv(states: torch.Tensor, repeats: int) -> torch.Tensor:
    """GQA head expansion (``reference.py:10-15``): ``[B, n_kv, T, D] -> [B, n_kv * repeats, T, D]``
    with query head ``i`` reading kv head ``i // repeats``."""
    return states if repeats == 1 else torch.repeat_interleave(states, repeats, dim=1)


def _causal_mask(query_len: int, key_len: int, device) -> torch.Tensor | None:
    """Additive float mask of ``query_len`` queries that are the last ``query_len`` of
    ``key_len`` keys (``reference.py:18-27``): query ``i`` sees keys ``0 .. key_len -
    query_len + i``; None for one query."""
    if query_len == 1:
        return None
    last_visible = torch.arange(query_len, device=device)[:, None] + (key_len - query_len)
    hidden = torch.arange(key_len, device=device)[None, :] > last_visible
    return torch.zeros(query_len, key_len, device=device).masked_fill(hidden, float("-inf"))


def reference_attention(manager, layer_idx: int, query: torch.Tensor, key_new: torch.Tensor,
                        value_new: torch.Tensor, scaling: float) -> torch.Tensor:
    """Dense path on the device (``reference.py:30-56``), for every sequence of the batch.

    ``query [B, n_q, q_len, D]``; ``key_new/value_new [B, n_kv, q_len, D]``.
    History is dequantised by the HIP kernel; attention is float32.
    """
    layer = manager.layers[layer_idx]
    layer.flush()  # deferred residual pages of this layer, if any
    if query.shape[0] != layer.batch:
        raise ValueError(f"query batch {query.shape[0]} != cache batch {layer.batch}")
    if not query.is_cuda:
        raise RuntimeError("logitfill_amd runs on ROCm devices only (there is no CPU path)")
    repeats = manager.n_q // manager.n_kv
    tail_k, tail_v = layer.tail_buffers()
    outs = []
    for b in range(layer.batch):
        key_hist, value_hist = layer.dequantize(b)
        pieces_k, pieces_v = [key_hist], [value_hist]
        tl = layer.tail_lens[b]
        if tl:
            pieces_k.append(tail_k[b, :, :tl].float())
            pieces_v.append(tail_v[b, :, :tl].float())
        pieces_k.append(key_new[b].float())
        pieces_v.append(value_new[b].float())
        key = repeat_kv(torch.cat(pieces_k, dim=1).unsqueeze(0), repeats)[0].contiguous()
        value = repeat_kv(torch.cat(pieces_v, dim=1).unsqueeze(0), repeats)[0].contiguous()
        q = query[b].float().contiguous()                                  # [n_q, q_len, D]
        scores = torch.matmul(q, key.transpose(1, 2).contiguous()) * scaling
        mask = _causal_mask(q.shape[1], key.shape[1], q.device)
        if mask is not None:
            scores = scores + mask
        probs = torch.softmax(scores, dim=-1)
        outs.append(torch.matmul(probs, value))
    return torch.stack(outs).to(dtype=query.dtype)


_CU_COUNT: dict = {}


def _cu_count(device) -> int:
    key = str(device)
    if key not in _CU_COUNT:
        _CU_COUNT[key] = int(torch.cuda.get_device_properties(device).multi_processor_count)
    return _CU_COUNT[key]


# Decode time of one sequence's residual (the BF16 tail page and the new token) in packed
# pages, for balancing the split-K items: a fixed part (the residual pass's load round, its
# matrix-core page and the merge of its wave partials) and a part that grows with the tail, taken
# from the batch's longest tail (lf_plan_decode takes one cost for every sequence).  Measured with
# the cost forced, 28 layers: c2 (100-token tails) 88.5-89.0 us per layer-step for 2-8 pages and
# 90.5 at 1; c1 (37-token tails, 3-page items) 24.2-24.4 us for 2-8 pages, best from 3 up (the
# residual is then an item of its own).
RESIDUAL_FIXED_PAGES = 3
RESIDUAL_TAIL_PAGES = 1  # added for a tail of 64 tokens or more


def residual_pages(tail_lens) -> int:
    """Residual cost in pages for the longest of ``tail_lens``: 3 + round(tail / 127)."""
    t = min(max(max(tail_lens, default=0), 0), 127)
    return RESIDUAL_FIXED_PAGES + (RESIDUAL_TAIL_PAGES * t + 63) // 127


# Fixed cost of one split-K item, in packed pages: the workgroup's prologue (argument block, work
# record, DMA set-up, q and tier table: the first page's barrier passes ≈8 us after the start on
# c2 and c1, per-workgroup stamps), its epilogue (≈1.6 us) and its share of the cross-split reduce,
# against 1.7-2.2 us per page.
ITEM_OVERHEAD_PAGES = 5
# A workgroup with a CU to itself (a launch of at most one workgroup per CU) runs its pages and
# its fixed cost this much faster than two sharing a CU.  Fitted to c1 (8 x 64 pages + a
# 37-token residual, 2 kv heads): 5-page items (224 workgroups, one per CU) 19.7-19.8 us per
# layer-step against 20.0-20.2 for the one-round 3-page items (368), 21.0 for 4 pages (272:
# some share) and 20.9-26 for 6-10 pages (same-process comparison).
ALONE_FACTOR = 0.78


@functools.lru_cache(maxsize=256)
def _pages_per_split(pages: tuple, n_kv: int, residual_pages: int, slots: int) -> int:
    p = np.asarray(pages, dtype=np.int64)
    work = p + residual_pages
    top = max(1, -(-n_kv * int(work.sum()) // slots))
    # sizes above the one-round size leave slots empty: worth it only when every workgroup then
    # has a CU to itself
    size = np.arange(max(top, int(work.max())), 0, -1, dtype=np.int64)[:, None]   # largest first
    items = np.where(p[None, :] == 0, 1, -(-work[None, :] // size))   # lf_plan_decode's count
    wgs = n_kv * items.sum(axis=1)
    rounds = -(-wgs // slots)
    largest = (-(-work[None, :] // items)).max(axis=1)
    cost = (rounds * (largest + ITEM_OVERHEAD_PAGES)).astype(np.float64)
    alone = wgs <= slots // 2
    cost = np.where(alone, (largest + ITEM_OVERHEAD_PAGES) * ALONE_FACTOR, cost)
    cost = np.where((size[:, 0] > top) & ~alone, np.inf, cost)
    return int(size[int(np.argmin(cost)), 0])                          # ties: fewest items


def choose_pages_per_split(hist_pages: list[int], n_kv: int, residual_pages: int, device=None) -> int:
    """Work per split-K item, in pages.  The decode kernel holds two workgroups per CU (the
    slots).  Items of ``total work / slots`` pages fill the slots once when every sequence's
    work (its pages plus its residual) divides evenly; with ragged lengths the per-sequence
    rounding makes more items than slots, and the excess runs as a second round of full-size
    items.  The size is therefore the one, up to that one-round size, that minimises
    rounds x (largest item + the per-item cost), with ties going to fewer items -- or a larger
    size whose items leave every workgroup a CU of its own, when that costs less at
    ``ALONE_FACTOR`` (small batches: c1 takes 5-page items instead of 3)."""
    forced = env_int("LOGITFILL_AMD_PAGES_PER_SPLIT", 0)
    if forced > 0:
        return forced
    slots = 2 * (_cu_count(device) if device is not None else 256)
    return _pages_per_split(tuple(int(x) for x in hist_pages), int(n_kv), int(residual_pages), slots)


# Of the two decode workgroups that share a CU, the one dispatched second runs this much slower
# (measured on c2: 72 against 88 us for equal items; the hardware issues the older waves first).
LATE_SLOWDOWN = 1.22


def age_split(hist_pages: list[int], n_kv: int, residual_pages: int, pages_per_split: int, cus: int):
    """Per-sequence split sizes that give the earlier-dispatched workgroups the larger items,
    or None to keep ``pages_per_split`` for every sequence.

    The decode kernel dispatches its work list item-major (workgroup item * n_kv + h), two
    workgroups per CU: the first ``cus`` workgroups each get a CU of their own and the rest
    share one with them, running ``LATE_SLOWDOWN`` times slower.  For a batch of equal
    sequences whose plan fills that one round (at least 90 % of the slots), the first s
    sequences are cut into k_o items and the others into k_y, the (s, k_o, k_y) that minimises
    the slowest item's estimated time (size x 1, or x LATE_SLOWDOWN for a sequence whose items
    reach past the first ``cus`` workgroups) within the round, if that beats the uniform split.
    c2 (16 x 260 pages of work, 4 kv heads): 8 sequences of 7 items and 8 of 9 instead of 16 of
    8, 88.6 -> 85.2 us."""
    r = _age_split(tuple(int(p) for p in hist_pages), int(n_kv), int(residual_pages), int(pages_per_split), int(cus))
    return None if r is None else list(r)


@functools.lru_cache(maxsize=256)
def _age_split(hist_pages: tuple, n_kv: int, residual_pages: int, pages_per_split: int, cus: int):
    B = len(hist_pages)
    if B < 2 or len(set(hist_pages)) != 1 or hist_pages[0] <= 0 or n_kv <= 0 or pages_per_split <= 0:
        return None
    work = hist_pages[0] + residual_pages
    positions = 2 * cus // n_kv      # item positions in one round
    first = cus // n_kv              # positions whose workgroups have a CU to themselves
    k0 = -(-work // pages_per_split)
    if B * k0 > positions or B * k0 * n_kv < 0.9 * 2 * cus:
        return None

    def cost(s, ko, ky):
        # sequences 0..s-1 hold items [0, s ko), the others [s ko, s ko + (B - s) ky): a group
        # is slowed when its last item lies past the first ``first`` positions
        total = s * ko + (B - s) * ky
        t_old = -(-work // ko) * (LATE_SLOWDOWN if s * ko > first else 1.0) if s else 0.0
        t_young = -(-work // ky) * (LATE_SLOWDOWN if total > first else 1.0) if s < B else 0.0
        return max(t_old, t_young)

    # the two sizes differ by about LATE_SLOWDOWN at the optimum: counts within 1.5x of k0
    best = (cost(0, k0, k0), 0, k0, k0)
    for s in range(1, B):
        for ko in range(max(1, (2 * k0) // 3), k0 + 1):
            for ky in range(k0, (3 * k0 + 1) // 2 + 1):
                if s * ko + (B - s) * ky > positions:
                    break
                c = cost(s, ko, ky)
                if c < best[0] - 1e-9:
                    best = (c, s, ko, ky)
    _, s, ko, ky = best
    if s == 0:
        return None
    counts = [ko] * s + [ky] * (B - s)
    sizes = tuple(-(-work // k) for k in counts)
    # lf_plan_decode cuts ceil(work / size) items: the sizes must give the chosen counts back
    if any(-(-work // z) != k for z, k in zip(sizes, counts)):
        return None
    return sizes


# Share of a CU's two items that goes to the workgroup dispatched first (the older wave of a
# SIMD issues first, so that workgroup runs ahead of its partner); measured on c2 by timing
# the paired plan at first-item sizes 33..39 pages of a 65-page pair: 36-37 best (67.8 us
# against 69.9 for the two-size split).
PAIR_FIRST_SHARE = 0.56
# Small batches (the uniform plan leaves each workgroup a CU to itself, the prologue
# dominates): the first items take this share of a CU's pages and the rest follow as 2-page
# items, the residual as an item of its own.  Measured on c1 (8 x 64 pages, 2 kv heads, 256
# CUs): first items of 3 pages + 2-page items 18.02 us against 19.32 for the uniform 5-page
# plan; 4-page first items and no second items 18.28; 3 + 3-4 pages 20.26; the residual on
# the last 2-page item 22.72; more than two workgroups per CU 24.5-25.6.
SMALL_FIRST_SHARE = 0.75
SMALL_SECOND_PAGES = 2


def paired_split(hist_pages: list[int], n_kv: int, residual_pages: int, cus: int, pages_per_split: int):
    """("paired", first_size, second_size) for a batch of equal sequences whose items can pair
    up on the CUs, or None.  Every sequence gets k = cus / (batch x n_kv) first items of
    ``first_size`` pages, listed (dispatched) before any other item, one workgroup per CU:
      - second_size 0 (the uniform plan ``pages_per_split`` fills one round of two workgroups
        per CU): k second items share the rest, the residual on the last; both workgroups of
        a CU finish together;
      - second_size > 0 (the uniform plan leaves every workgroup a CU of its own): the rest in
        items of second_size pages and the residual as an item of its own.
    See ``paired_plan``."""
    B = len(hist_pages)
    if B < 1 or n_kv <= 0 or cus <= 0 or pages_per_split <= 0 or len(set(hist_pages)) != 1 or hist_pages[0] <= 0:
        return None
    if cus % (B * n_kv):
        return None
    k = cus // (B * n_kv)
    P = int(hist_pages[0])
    work = P + int(residual_pages)
    k0 = -(-work // int(pages_per_split))        # the uniform plan's items per sequence
    wgs = B * n_kv * k0
    if 0.9 * 2 * cus <= wgs <= 2 * cus:
        first = int(round(PAIR_FIRST_SHARE * work / k))
        rest = work - k * first                    # the second items' work, residual included
        # every second item keeps at least a page, the last one (which takes the residual) too
        if first < 1 or rest // k - residual_pages < 1:
            return None
        return ("paired", first, 0)
    if wgs <= cus and k >= 2:
        first = max(1, int(round(SMALL_FIRST_SHARE * P / k)))
        rest = P - k * first
        if rest < 0:
            return None
        n_second = -(-rest // SMALL_SECOND_PAGES)
        if B * n_kv * (k + n_second + 1) > 2 * cus:
            return None
        return ("paired", first, SMALL_SECOND_PAGES)
    return None


def paired_plan(hist_pages: list[int], k: int, first: int, residual_pages: int,
                second: int = 0) -> tuple[list[int], list[int]]:
    """Work list and seq_work of a paired plan: the k first items of every sequence, then every
    sequence's other items (list order = dispatch order), each item's partial slot in its kind
    field (bits 8.. = slot + 1) so that each sequence's partials take consecutive slots.
    ``second`` 0: k second items sharing the rest of the work, the residual riding on the last
    (kind 2); ``second`` > 0: the rest in items of ``second`` pages, then a residual-only item
    (kind 1)."""
    B = len(hist_pages)
    if k < 1 or first < 1 or second < 0:
        raise ValueError("paired plan needs k >= 1 first items of >= 1 page")
    firsts, others, counts = [], [], []
    for b in range(B):
        P = int(hist_pages[b])
        if second == 0:
            rest = P + residual_pages - k * first
            sizes = [rest // k + (1 if j < rest % k else 0) for j in range(k)]
            sizes[-1] -= residual_pages
        else:
            rest = P - k * first
            sizes = [min(second, rest - second * j) for j in range(-(-rest // second))] if rest > 0 else []
        if sizes and min(sizes) < 1 or P < k * first:
            raise ValueError("paired plan leaves an item without a page")
        n = k + len(sizes) + (1 if second else 0)
        base = sum(counts)
        counts.append(n)
        p = 0
        for j in range(k):
            firsts.append((b, p, p + first, 0, base + j))
            p += first
        for j, z in enumerate(sizes):
            kind = 2 if second == 0 and j == len(sizes) - 1 else 0
            others.append((b, p, p + z, kind, base + k + j))
            p += z
        if second:
            others.append((b, p, p, 1, base + n - 1))
        if p != P:
            raise ValueError("paired plan does not cover the history")
    work = []
    for b, p0, p1, kind, slot in firsts + others:
        work += [b, p0, p1, kind | ((slot + 1) << 8)]
    seq = []
    base = 0
    for n in counts:
        seq += [base, n]
        base += n
    return work, seq


def plan_work(hist_pages: list[int], sizes: list[int], residual_pages: int) -> tuple[list[int], list[int]]:
    """Host work list (b, page0, page1, kind) x n and per-sequence (first, count) for
    per-sequence split sizes.  The sequences go into the list (the decode kernel's dispatch
    order) by decreasing item size -- larger items first, the smaller ones filling the last
    round (c4: 376.6 -> 371.7 us) -- ties in batch order; each run of consecutive sequences
    with one size is planned by one lf_plan_decode call, its sequence and item indices
    shifted into place."""
    lib = _native.load()
    batch = len(hist_pages)
    if len(sizes) != batch:
        raise ValueError("one split size per sequence")

    def item_pages(b):
        w = int(hist_pages[b]) + residual_pages
        return w / (1 if hist_pages[b] == 0 else -(-w // int(sizes[b])))

    order = sorted(range(batch), key=lambda b: -item_pages(b))
    work, seq = [], [0] * (2 * batch)
    r0 = 0
    while r0 < batch:
        r1 = r0
        while r1 < batch and sizes[order[r1]] == sizes[order[r0]]:
            r1 += 1
        run = order[r0:r1]
        m = len(run)
        size = int(sizes[run[0]])
        pages = [int(hist_pages[b]) for b in run]
        cap = sum(-(-(p + residual_pages) // size) for p in pages) + m
        w = (ctypes.c_int32 * (4 * cap))()
        sq = (ctypes.c_int32 * (2 * m))()
        n = lib.lf_plan_decode((ctypes.c_int32 * m)(*pages), m, size, residual_pages, w, cap, sq)
        if n < 0:
            _native.check(n, "lf_plan_decode")
        base = len(work) // 4
        for i in range(n):
            work += [run[w[4 * i]], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]]
        for i, b in enumerate(run):
            seq[2 * b], seq[2 * b + 1] = base + sq[2 * i], sq[2 * i + 1]
        r0 = r1
    return work, seq


class DecodePlan:
    """Device work list for one layer's current history lengths (rebuilt when they change).
    ``pages_per_split``: one size for every sequence, a tuple of per-sequence sizes, or
    ("paired", first_size, second_size) for ``paired_plan`` on the device's CU count."""

    def __init__(self, hist_pages: list[int], n_kv: int, pages_per_split, device, residual_pages: int,
                 cus: int | None = None):
        batch = len(hist_pages)
        if isinstance(pages_per_split, tuple) and pages_per_split and pages_per_split[0] == "paired":
            if cus is None:
                cus = _cu_count(device)
            work, seq = paired_plan(list(hist_pages), cus // (batch * n_kv), int(pages_per_split[1]),
                                    residual_pages, int(pages_per_split[2]))
            self.key = (tuple(hist_pages), pages_per_split, residual_pages)
        else:
            sizes = [pages_per_split] * batch if isinstance(pages_per_split, int) else list(pages_per_split)
            work, seq = plan_work(list(hist_pages), sizes, residual_pages)
            self.key = (tuple(hist_pages), pages_per_split if isinstance(pages_per_split, int) else tuple(sizes),
                        residual_pages)
        self.n_work = len(work) // 4
        self.work = _native.upload(work, torch.int32, device)
        self.seq_work = _native.upload(seq, torch.int32, device)
        # host copies: a small plan travels in the kernels' arguments (lf_decode_args.work_host)
        self.work_host = np.ascontiguousarray(work, dtype=np.int32)
        self.seq_work_host = np.ascontiguousarray(seq, dtype=np.int32)
        self.pages_per_split = pages_per_split


def _expect(t: torch.Tensor, shape, name: str) -> None:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_cuda:
        raise RuntimeError(f"{name} is on {t.device}; logitfill_amd runs on ROCm devices only")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def kernel_choice() -> int:
    """``LOGITFILL_AMD_KERNEL``: auto (default), valu or mfma."""
    name = os.environ.get("LOGITFILL_AMD_KERNEL", "auto").lower()
    return {"auto": _native.KERNEL_AUTO, "valu": _native.KERNEL_VALU, "mfma": _native.KERNEL_MFMA}[name]


def decode_into(manager, layer_idx: int, query: torch.Tensor, key_new, value_new, scaling: float,
                out: torch.Tensor, kernel: int | None = None, pages_per_split: int | None = None,
                noalloc: bool = False, commit: bool = False) -> bool:
    """Enqueue the fused decode kernel for layer ``layer_idx`` writing ``out``.

    One new token: ``query/out [B, n_q, D]``, ``key_new/value_new [B, n_kv, D]`` or None.
    ``q_len`` new tokens: ``query/out [B, n_q, q_len, D]``, ``key_new/value_new
    [B, n_kv, q_len, D]``; query token j sees the history, the tail and new tokens 0..j
    (reference ``reference.py:18-27,48``).  Everything is enqueued on the current stream;
    nothing synchronises.  ``noalloc`` calls ``lf_decode_attention_noalloc`` (the partials in
    the library's per-GPU scratch array instead of the manager's workspace).

    ``commit``: also append the new tokens to the layer, in the same launch
    (``lf_decode_args.commit_new``), when no residual page fills; returns whether it did --
    when it did not, the caller commits as usual (``PackedKVManager.commit``).
    """
    layer = manager.layers[layer_idx]
    layer.flush()  # deferred residual pages of this layer, if any
    B, D = layer.batch, layer.head_dim
    qshape = query.shape
    q_len = int(qshape[2]) if len(qshape) == 4 else 1
    tok = (q_len,) if len(qshape) == 4 else ()
    want_q = (B, manager.n_q, *tok, D)
    if qshape != want_q or out.shape != want_q:
        _expect(query, want_q, "query")
        _expect(out, want_q, "out")
    if key_new is not None:
        want_kv = (B, manager.n_kv, *tok, D)
        if key_new.shape != want_kv or value_new.shape != want_kv:
            _expect(key_new, want_kv, "key_new")
            _expect(value_new, want_kv, "value_new")
    kernel = kernel_choice() if kernel is None else kernel
    P = layer.page_size
    hist_pages = tuple(h // P for h in layer.hist_lens)
    # q_len new tokens lengthen the residual (a chunk of 128 tokens more past a full page)
    res_pages = residual_pages(layer.tail_lens) + (max(layer.tail_lens, default=0) + q_len - 1) // P * (
        RESIDUAL_FIXED_PAGES + RESIDUAL_TAIL_PAGES)
    # workgroups per (item, kv head): one per tile of query rows
    tiles = -(-(manager.n_q // manager.n_kv * q_len) // MFMA_TILE_ROWS)
    if pages_per_split is None:
        # the split depends on the history, the residual cost, the environment's override and
        # whether the matrix-core kernel's dispatch order applies: chosen again when one changes
        age = kernel != _native.KERNEL_VALU and tiles == 1
        choice_key = (hist_pages, res_pages, os.environ.get("LOGITFILL_AMD_PAGES_PER_SPLIT"), age, tiles)
        cached = layer.__dict__.get("_lf_split_choice")
        if cached is None or cached[0] != choice_key:
            size = choose_pages_per_split(list(hist_pages), layer.n_kv * tiles, res_pages, layer.device)
            if age and choice_key[2] is None:
                cus = _cu_count(layer.device)
                paired = paired_split(list(hist_pages), layer.n_kv, res_pages, cus, size)
                if paired is not None:
                    size = paired
                else:
                    sizes = age_split(list(hist_pages), layer.n_kv, res_pages, size, cus)
                    size = size if sizes is None else tuple(sizes)
            cached = (choice_key, size)
            layer.__dict__["_lf_split_choice"] = cached
        pages_per_split = cached[1]
    plan = layer.decode_plan
    if plan is None or plan.key != (hist_pages, pages_per_split, res_pages):
        # the layers of a manager share their history lengths, so one plan serves them all (its
        # device lists are only read): built by the first layer after a change, found by the rest
        shared = manager.__dict__.setdefault("_lf_plans", {})
        pkey = (hist_pages, pages_per_split, res_pages, layer.n_kv, str(layer.device))
        plan = shared.get(pkey)
        if plan is None:
            if len(shared) >= 8:
                shared.clear()
            plan = DecodePlan(list(hist_pages), layer.n_kv, pages_per_split, layer.device, res_pages)
            shared[pkey] = plan
        layer.decode_plan = plan
    lib = _native.load()
    wkey = (manager.n_q * q_len, layer.head_dim)
    ws_need = plan.__dict__.get("_lf_ws_bytes")
    if ws_need is None or ws_need[0] != wkey:
        ws_need = (wkey, lib.lf_decode_workspace_bytes(wkey[0], wkey[1], plan.n_work))
        plan.__dict__["_lf_ws_bytes"] = ws_need
    ws = None if noalloc else manager.workspace(ws_need[1])
    tail_k, tail_v = layer.tail_buffers()
    if key_new is not None and value_new.dtype != key_new.dtype:
        raise TypeError("key_new and value_new must share a dtype")
    tail_len = layer.tail_len_device()
    # Every field but the four per-call tensors is fixed while the plan, the buffers and the
    # call's settings stay the same: the argument block is kept on the layer and reused.  The
    # buffers are compared by identity (each one's pointer is fixed for its lifetime; the cache
    # entry holds them, so an id cannot be reused while it is kept).
    held = (plan, ws, tail_k, tail_v, tail_len)
    static_key = (id(plan), id(ws), id(tail_k), id(tail_v), id(tail_len), query.dtype, out.dtype,
                  None if key_new is None else key_new.dtype, manager.n_q, float(scaling), kernel, q_len)
    cached_args = layer.__dict__.get("_lf_decode_args")
    if cached_args is not None and cached_args[0] == static_key:
        a = cached_args[1]
    else:
        a = _native.DecodeArgs()
        a.q_dtype = _native.dtype_code(query.dtype)
        if key_new is not None:
            a.new_dtype = _native.dtype_code(key_new.dtype)
        if tail_k is not None:
            a.tail_k = tail_k.data_ptr()
            a.tail_v = tail_v.data_ptr()
            a.tail_dtype = _native.dtype_code(tail_k.dtype)
            a.tail_cap = int(tail_k.shape[2])
        else:
            a.tail_dtype = _native.LF_BF16
            a.tail_cap = 0
        a.tail_len = tail_len.data_ptr()
        a.out_dtype = _native.dtype_code(out.dtype)
        a.n_q = manager.n_q
        a.scaling = float(scaling)
        a.work = plan.work.data_ptr()
        a.n_work = plan.n_work
        a.seq_work = plan.seq_work.data_ptr()
        a.work_host = plan.work_host.ctypes.data
        a.seq_work_host = plan.seq_work_host.ctypes.data
        a.workspace = 0 if ws is None else ws.data_ptr()
        a.workspace_bytes = 0 if ws is None else ws.numel()
        a.kernel = kernel
        a.q_len = q_len
        layer.__dict__["_lf_decode_args"] = (static_key, a, held)
    a.query = query.data_ptr()
    a.out = out.data_ptr()
    a.k_new = 0 if key_new is None else key_new.data_ptr()
    a.v_new = 0 if key_new is None else value_new.data_ptr()
    # the commit folds into the launch while every sequence's residual page stays below full
    fold = commit and key_new is not None and tail_k is not None and max(layer.tail_lens) + q_len < P
    a.commit_new = 1 if fold else 0
    stream = _native.current_stream_ptr(layer.device)
    if noalloc:
        st = lib.lf_decode_attention_noalloc(layer.layer_struct(), a, stream)
        _native.check(st, "lf_decode_attention_noalloc")
    else:
        st = lib.lf_decode_attention(layer.layer_struct(), a, stream)
        _native.check(st, "lf_decode_attention")
    if fold:
        layer.tail_lens = [t + q_len for t in layer.tail_lens]
    return fold


def _kernel_attention(manager, layer_idx: int, query: torch.Tensor, key_new: torch.Tensor,
                      value_new: torch.Tensor, scaling: float, commit: bool = False):
    """Decode through the HIP kernels (replaces ``reference.py:59-109``).  The tensors go to
    ``decode_into`` in their ``[B, heads, q_len, D]`` form (for one token the same memory as
    ``[B, heads, D]``), copied only when not contiguous: this runs once per layer and step.
    Returns (output, whether the commit was folded into the launch)."""
    B, n_q, q_len, D = query.shape
    q = query if query.is_contiguous() else query.contiguous()
    kn = key_new if key_new.is_contiguous() else key_new.contiguous()
    vn = value_new if value_new.is_contiguous() else value_new.contiguous()
    out = torch.empty(B, n_q, q_len, D, dtype=query.dtype, device=query.device)
    folded = decode_into(manager, layer_idx, q, kn, vn, scaling, out, commit=commit)
    return out, folded


# Query rows per workgroup of the matrix-core decode kernel: rows beyond it ((n_q / n_kv) * q_len
# per kv head) run as further row tiles, each a workgroup of its own over the same pages.
MFMA_TILE_ROWS = 8


def valu_tile_rows(head_dim: int) -> int:
    """Query rows per workgroup of the general decode kernel (8 at head_dim 1024, else 16)."""
    return 8 if head_dim > 512 else 16

# Calls that took the dense dequantise-then-attend path because the decode kernels do not
# serve their shape, by reason (read by tests and benchmarks; see ``packed_attention``).
DENSE_FALLBACKS: Counter = Counter()
_WARNED: set = set()


def kernel_unsupported_reason(manager, q_len: int = 1) -> str | None:
    """Why ``lf_decode_attention`` would not serve this manager's shape, or None when it does
    (the checks of the C entry point: int2 Values as the reference kernel requires,
    ``reference.py:62``; head_dim a power of two in 8..1024, as the reference kernel takes,
    ``kernel.cu:224-230``; at most 64 Value groups; the general kernel's LDS within 160 KB).
    Any number of query rows per kv head is served: the kernels tile them across workgroups."""
    D = int(manager.head_dim)
    if manager.bit_v != 2:
        return f"bit_v={manager.bit_v} (the decode kernels take int2 Values)"
    if D < 8 or D > 1024 or D & (D - 1):
        return f"head_dim={D} (the decode kernels take powers of two in 8..1024)"
    vg = D // int(manager.v_group_size)
    if vg > 64:
        return f"{vg} Value groups per token (at most 64)"
    slots = max(sum(layer.widths) for layer in manager.layers) if manager.layers else D
    G = valu_tile_rows(D)
    lds = 4 * (G * D + G * 64 + 2 * 64 * vg + 64 * -(-D // 16) + G * slots)
    if lds > 160 * 1024:
        return f"{lds} bytes of LDS for the general kernel (at most 160 KB)"
    return None


def packed_attention(manager, layer_idx: int, query: torch.Tensor, key_new: torch.Tensor,
                     value_new: torch.Tensor, scaling: float, *, commit: bool = False) -> torch.Tensor:
    """``reference.py:112-116``: ``query [B, n_q, q_len, D]`` -> ``[B, n_q, q_len, D]``.

    Shapes the decode kernels serve run the HIP split-K decode.  Others take the dense
    dequantise-then-attend path on the device, as the reference falls back to its dense path
    (``reference.py:62-68,105-108``) -- but not silently: each fallback is counted in
    ``DENSE_FALLBACKS``, warned about once per reason, and raises instead when the environment
    sets ``LOGITFILL_AMD_STRICT=1``.

    ``commit`` (extension, keyword only): also append ``key_new / value_new`` to the layer,
    as ``manager.commit(layer_idx, key_new, value_new)`` right after the call would (the
    reference model's order, ``qwen2_attention.py:223-256``).  While no residual page fills
    the append runs inside the decode launch (one launch per layer fewer); otherwise, and on
    the dense path, through ``manager.commit``.
    """
    if not query.is_cuda:
        raise RuntimeError("logitfill_amd runs on ROCm devices only (there is no CPU path)")
    q_len = int(query.shape[-2])
    cache = manager.__dict__.setdefault("_lf_kernel_reason", {})  # the shape is fixed per manager
    if q_len not in cache:
        cache[q_len] = kernel_unsupported_reason(manager, q_len)
    reason = cache[q_len]
    if reason is None:
        out, folded = _kernel_attention(manager, layer_idx, query, key_new, value_new, scaling, commit)
        if commit:
            if not folded:
                manager.commit(layer_idx, key_new, value_new)
            elif layer_idx == len(manager.layers) - 1:
                manager.seq_len = manager.layers[layer_idx].length
        return out
    if os.environ.get("LOGITFILL_AMD_STRICT", "") == "1":
        raise _native.LFError(_native.LF_E_UNSUPPORTED, reason, "packed_attention")
    DENSE_FALLBACKS[reason] += 1
    if reason not in _WARNED:
        _WARNED.add(reason)
        warnings.warn(f"packed_attention: {reason}; running the dense dequantise-then-attend path on the device",
                      RuntimeWarning, stacklevel=2)
    out = reference_attention(manager, layer_idx, query, key_new, value_new, scaling)
    if commit:
        manager.commit(layer_idx, key_new, value_new)
    return out
