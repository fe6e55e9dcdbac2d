"""Seeded synthetic inputs for the packed decode path (tests and benchmarks).

Distributions (one independent draw per layer, seed = base + layer):

* tier table ``[n_kv, D]``: i.i.d. levels with P(int2, int4, int8, fp16) =
  (0.60, 0.25, 0.10, 0.05); then, per head, random one-step downgrades while
  the extra Key bits exceed the budget and random one-step upgrades (int2 ->
  int4 first, then any level whose step still fits) until they equal it.
  The budget is the reference allocator's rule: ``target_bit_k = 2*target_bit
  - bit_v`` and ``extra = round((target_bit_k - 2) * D)`` bits above the int2
  floor, with step costs int2->int4 2, int4->int8 4, int8->fp16 8
  (reference ``src/logitfill/allocators/allocate.py:14-53``);
* Key ``K[h, t, c] = N(0,1) * sigma[h, c]``, ``sigma ~ LogNormal(0, 1)`` per
  (kv head, channel), 4 outlier channels per head (uniform, without
  replacement) with sigma x 20; ``V ~ N(0, 1)``; ``Q ~ N(0, 1) / sqrt(D)``;
  all rounded to bf16.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

LEVEL_EXTRA = np.array([0, 2, 6, 14], dtype=np.int64)   # extra bits above int2 per level
LEVEL_BITS = np.array([2, 4, 8, 16], dtype=np.int64)
STEP_COST = np.array([2, 4, 8], dtype=np.int64)          # cost of level l -> l+1


def key_budget(target_bit: float, bit_v: int = 2, head_dim: int = 128) -> int:
    """Extra Key bits per head above the int2 floor (reference ``allocate.py:14-53``)."""
    target_k = 2.0 * float(target_bit) - float(bit_v)
    if target_k < 2.0 or target_k > 16.0:
        raise ValueError(f"target_bit {target_bit} with bit_v {bit_v} gives Key target {target_k}")
    return int(round((target_k - 2.0) * head_dim))


def sample_tier_levels(n_kv: int, head_dim: int, target_bit: float, seed: int, bit_v: int = 2) -> np.ndarray:
    """Seeded tier table ``[n_kv, head_dim]`` int64 whose every head spends exactly the budget."""
    rng = np.random.default_rng(seed)
    budget = key_budget(target_bit, bit_v, head_dim)
    if budget > int(LEVEL_EXTRA[3]) * head_dim:
        raise ValueError("budget exceeds an all-fp16 head")
    levels = rng.choice(4, size=(n_kv, head_dim), p=[0.60, 0.25, 0.10, 0.05]).astype(np.int64)
    for h in range(n_kv):
        row = levels[h]
        spent = int(LEVEL_EXTRA[row].sum())
        while spent > budget:
            c = int(rng.choice(np.nonzero(row > 0)[0]))
            row[c] -= 1
            spent -= int(STEP_COST[row[c]])
        while spent < budget:
            gap = budget - spent
            cand = np.nonzero(row == 0)[0] if gap >= 2 else np.array([], dtype=np.int64)
            if cand.size == 0:
                cand = np.nonzero((row < 3) & (STEP_COST[np.minimum(row, 2)] <= gap))[0]
            if cand.size == 0:
                break
            c = int(rng.choice(cand))
            spent += int(STEP_COST[row[c]])
            row[c] += 1
        levels[h] = row
    return levels


@dataclass
class LayerData:
    levels: np.ndarray        # [n_kv, D] int64
    key: torch.Tensor         # [B, n_kv, T, D] bf16
    value: torch.Tensor       # [B, n_kv, T, D] bf16
    query: torch.Tensor       # [B, n_q, D] bf16
    key_new: torch.Tensor     # [B, n_kv, D] bf16
    value_new: torch.Tensor   # [B, n_kv, D] bf16


def channel_sigma(n_kv: int, head_dim: int, gen: torch.Generator, outliers: int = 4) -> torch.Tensor:
    """Per (kv head, channel) Key scale: LogNormal(0,1), ``outliers`` channels per head x 20."""
    sigma = torch.exp(torch.randn(n_kv, head_dim, generator=gen))
    for h in range(n_kv):
        idx = torch.randperm(head_dim, generator=gen)[:outliers]
        sigma[h, idx] *= 20.0
    return sigma


def make_layer(batch: int, n_q: int, n_kv: int, head_dim: int, tokens: int, target_bit: float, seed: int,
               device="cpu", dtype=torch.bfloat16, bit_v: int = 2) -> LayerData:
    """One layer's seeded inputs.  ``tokens`` = history + residual tokens per sequence.

    The tier table, channel scales and outliers are drawn on the CPU; the
    Gaussian tensors are drawn with a generator on ``device`` (so large
    benchmark layers never touch host memory).  Same seed and device -> same data.
    """
    levels = sample_tier_levels(n_kv, head_dim, target_bit, seed, bit_v)
    cpu_gen = torch.Generator().manual_seed(int(seed))
    sigma = channel_sigma(n_kv, head_dim, cpu_gen).to(device)
    dev_gen = torch.Generator(device=device).manual_seed(int(seed) + 7919)
    key = torch.randn(batch, n_kv, tokens, head_dim, generator=dev_gen, device=device)
    key.mul_(sigma[None, :, None, :])
    key = key.to(dtype)
    value = torch.randn(batch, n_kv, tokens, head_dim, generator=dev_gen, device=device).to(dtype)
    query = (torch.randn(batch, n_q, head_dim, generator=dev_gen, device=device) / math.sqrt(head_dim)).to(dtype)
    knew = torch.randn(batch, n_kv, head_dim, generator=dev_gen, device=device)
    knew.mul_(sigma[None])
    key_new = knew.to(dtype)
    value_new = torch.randn(batch, n_kv, head_dim, generator=dev_gen, device=device).to(dtype)
    return LayerData(levels, key, value, query, key_new, value_new)


# BASELINE.json configurations (shapes only; tokens = history pages * 128 + residual).
CONFIGS = {
    "c0": dict(layers=1, batch=1, n_q=28, n_kv=4, head_dim=128, pages=8, residual=0, target_bit=2.5),
    "c1": dict(layers=28, batch=8, n_q=12, n_kv=2, head_dim=128, pages=64, residual=37, target_bit=2.5),
    "c2": dict(layers=28, batch=16, n_q=28, n_kv=4, head_dim=128, pages=256, residual=100, target_bit=2.5),
    "c2_k4": dict(layers=28, batch=16, n_q=28, n_kv=4, head_dim=128, pages=256, residual=100, target_bit=3.0),
    "c3": dict(layers=28, batch=64, n_q=28, n_kv=4, head_dim=128, pages=1, residual=0, target_bit=2.5),
    "c4": dict(layers=48, batch=32, n_q=40, n_kv=8, head_dim=128, pages=None, residual=None, target_bit=2.5),
}


def ragged_lengths(batch: int, seed: int, lo: int = 4096, hi: int = 65536, page: int = 128):
    """c4 contexts: uniform in [lo, hi] -> (full pages, residual 1..page-1) per sequence."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, size=batch)
    pages = ctx // page
    resid = rng.integers(1, page, size=batch)
    return [int(p) for p in pages], [int(r) for r in resid]
