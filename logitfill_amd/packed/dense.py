"""BF16 dense decode attention on the GPU: the comparator the packed path is measured against.

The reference has no dense decode kernel (its dense path is fp32 SDPA over the dequantised
history, ``src/logitfill/packed/reference.py:30-56``); this is the same single-query attention
over an uncompressed BF16 K/V cache, with the packed path's split-K skeleton
(``lf_dense_decode``), so ``bench.py`` can compare bytes and time at the same shape.
"""

from __future__ import annotations

import math

import torch

from logitfill_amd import _native

_PAGE = 128


def choose_tokens_per_split(batch: int, n_kv: int, tokens: int, device=None) -> int:
    """Tokens per split-K item: enough splits to fill two workgroups per CU once."""
    cus = int(torch.cuda.get_device_properties(device).multi_processor_count) if device is not None else 256
    splits = max(1, (2 * cus) // max(1, batch * n_kv))
    per = math.ceil(tokens / splits)
    return max(_PAGE, -(-per // _PAGE) * _PAGE)


def dense_decode(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, scaling: float,
                 out: torch.Tensor | None = None, tokens: int | None = None,
                 tokens_per_split: int | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Single-query attention of ``query [B, n_q, D]`` over ``key/value [B, n_kv, T, D]`` (bf16;
    any strides with unit channel stride) for the first ``tokens`` positions (default T).
    Returns ``out [B, n_q, D]`` bf16.  Enqueued on the current stream."""
    B, n_q, D = query.shape
    n_kv, T = key.shape[1], key.shape[2]
    tokens = T if tokens is None else tokens
    for name, t in (("query", query), ("key", key), ("value", value)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"{name} must be bfloat16, got {t.dtype}")
        if not t.is_cuda:
            raise RuntimeError(f"{name} is on {t.device}; logitfill_amd runs on ROCm devices only")
        if t.stride(-1) != 1:
            raise ValueError(f"{name} needs unit channel stride")
    if key.shape != value.shape or key.stride() != value.stride():
        raise ValueError("key and value must share shape and strides")
    if not query.is_contiguous():
        raise ValueError("query must be contiguous")
    if out is None:
        out = torch.empty((B, n_q, D), dtype=torch.bfloat16, device=query.device)
    tps = tokens_per_split or choose_tokens_per_split(B, n_kv, tokens, query.device)
    lib = _native.load()
    nbytes = lib.lf_dense_decode_workspace_bytes(B, n_kv, n_q, D, tokens, tps)
    if nbytes < 0:
        _native.check(int(nbytes), "lf_dense_decode_workspace_bytes")
    if workspace is None or workspace.numel() < nbytes:
        workspace = torch.empty(int(nbytes), dtype=torch.uint8, device=query.device)
    st = lib.lf_dense_decode(query.data_ptr(), key.data_ptr(), value.data_ptr(), B, n_q, n_kv, D, tokens,
                             key.stride(0), key.stride(1), key.stride(2), float(scaling), out.data_ptr(), tps,
                             workspace.data_ptr(), workspace.numel(), torch.cuda.current_stream().cuda_stream)
    _native.check(st, "lf_dense_decode")
    return out
