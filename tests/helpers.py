"""Shared helpers for the GPU parity tests: build the same inputs for the device
path and the CPU oracle, and compare results to the north-star bars."""
from __future__ import annotations

import numpy as np
import torch

from oracle import attention as oatt
from oracle import history as ohist

MAX_ABS = 2e-3      # decode output bar (bf16 output, fp32 accumulation)
REL_L2 = 1e-3


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def oracle_store(levels, key_b, value_b, page=128, kg=128, vg=128, bit_v=2):
    """Oracle page store of one sequence: ``key_b/value_b [n_kv, T, D]`` float32 values."""
    return ohist.pack_history(levels, key_b, value_b, page, kg, vg, bit_v)


def assert_history_equal(layer, b, store, *, tail=True):
    """Bit-exact equality of the device history of sequence ``b`` and an oracle store."""
    hk, hv = layer.export_reference(b)
    assert layer.hist_lens[b] == store.hist_len
    if store.hist_len == 0:
        assert hk is None
    else:
        for t in range(3):
            for name in ("code", "scale", "min"):
                ours = hk[t][name].cpu().numpy()
                ref = store.hist_k[t][name]
                assert ours.shape == ref.shape, (t, name, ours.shape, ref.shape)
                assert np.array_equal(ours.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), (t, name)
        ours16 = hk[3]["value"].cpu().numpy()
        assert ours16.shape == store.hist_k[3]["value"].shape
        assert np.array_equal(ours16.view(np.uint16), store.hist_k[3]["value"].view(np.uint16))
        for name in hv:
            ours = hv[name].cpu().numpy()
            ref = store.hist_v[name]
            assert ours.shape == ref.shape, (name, ours.shape, ref.shape)
            assert np.array_equal(ours.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), name
    if tail:
        tl = layer.tail_lens[b]
        assert tl == store.tail_len
        if tl:
            tk, tv = layer.tail_buffers()
            assert np.array_equal(f32(tk[b, :, :tl]), store.tail_k)
            assert np.array_equal(f32(tv[b, :, :tl]), store.tail_v)


def ulp(x: np.ndarray, dtype: str) -> np.ndarray:
    """Spacing of the output format at |x| (bf16: 8 significant bits, fp16: 11, fp32: 24)."""
    bits = {"bf16": 8, "fp16": 11, "fp32": 24}[dtype]
    ax = np.maximum(np.abs(x), np.finfo(np.float32).tiny)
    return np.exp2(np.floor(np.log2(ax)) - (bits - 1))


def decode_errors(ours: torch.Tensor, ref_fp32: np.ndarray, out_dtype="bf16"):
    """(max-abs, rel-L2, worst excess) of the device output against the oracle rounded to
    the output dtype.  ``excess`` is the largest |diff| among elements that are outside
    the max-abs bar *and* differ by more than one output ulp (a rounding flip of the
    output format is one ulp; for bf16 values above 0.5 one ulp already exceeds 2e-3)."""
    ref = oatt.round_to_dtype(ref_fp32.astype(np.float32), out_dtype).astype(np.float64)
    o = f32(ours).astype(np.float64).reshape(ref.shape)
    diff = np.abs(o - ref)
    max_abs = float(diff.max()) if diff.size else 0.0
    rel = float(np.linalg.norm(o - ref) / max(np.linalg.norm(ref), 1e-30))
    bad = (diff > MAX_ABS) & (diff > ulp(ref, out_dtype) * 1.0001)
    excess = float(diff[bad].max()) if bad.any() else 0.0
    return max_abs, rel, excess


def assert_decode_close(ours, ref_fp32, out_dtype="bf16", max_abs=MAX_ABS, rel_l2=REL_L2):
    """max-abs <= 2e-3 (or one output ulp, for outputs whose format
    resolution is coarser than the bar) and rel-L2 <= 1e-3, fp32 accumulation."""
    ref = oatt.round_to_dtype(ref_fp32.astype(np.float32), out_dtype).astype(np.float64)
    o = f32(ours).astype(np.float64).reshape(ref.shape)
    diff = np.abs(o - ref)
    rl = float(np.linalg.norm(o - ref) / max(np.linalg.norm(ref), 1e-30))
    bad = (diff > max_abs) & (diff > ulp(ref, out_dtype) * 1.0001)
    ma = float(diff.max()) if diff.size else 0.0
    assert not bad.any() and rl <= rel_l2, (
        f"max_abs={ma:.3g} (bar {max_abs} or 1 ulp; {int(bad.sum())} elements outside), "
        f"rel_l2={rl:.3g} (bar {rel_l2})")
    return ma, rl


def oracle_decode(store, query_b, key_new_b, value_new_b, scaling, n_q, n_kv):
    """float32 oracle output ``[n_q, D]`` for one sequence (one new token)."""
    out = oatt.reference_attention(store, query_b[:, None, :], key_new_b[:, None, :], value_new_b[:, None, :],
                                   scaling, n_q, n_kv)
    return out[:, 0, :]
