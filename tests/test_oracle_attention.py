"""Pin the oracle's dense decode path and page store.

References: src/logitfill/packed/reference.py:10-56 (repeat_kv, causal mask,
reference_attention) and src/logitfill/packed/cache.py:48-90 (append/flush).
Checks: float64 brute force, closed forms (one key -> its value; equal keys ->
mean of values; two keys with a known score gap), head mapping, mask geometry,
and page-store invariants.
"""
import math

import numpy as np
import pytest

from oracle import attention, history, layout

F32 = np.float32


def brute_attention(q, k, v, scale, mask=None):
    """Per-element float64 softmax attention, no vectorised tricks."""
    H, Q, D = q.shape
    T = k.shape[1]
    out = np.zeros((H, Q, D))
    for h in range(H):
        for i in range(Q):
            s = [scale * sum(float(q[h, i, c]) * float(k[h, t, c]) for c in range(D)) for t in range(T)]
            if mask is not None:
                s = [s[t] + float(mask[i, t]) for t in range(T)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            for c in range(D):
                out[h, i, c] = sum(w[t] * float(v[h, t, c]) for t in range(T)) / z
    return out


def test_sdpa_matches_bruteforce():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((3, 2, 8)).astype(F32)
    k = rng.standard_normal((3, 5, 8)).astype(F32)
    v = rng.standard_normal((3, 5, 8)).astype(F32)
    mask = attention.causal_mask(2, 5)
    assert np.allclose(attention.sdpa(q, k, v, 0.3, mask), brute_attention(q, k, v, 0.3, mask), atol=1e-6)
    assert np.allclose(attention.sdpa(q[:, :1], k, v, 0.3), brute_attention(q[:, :1], k, v, 0.3), atol=1e-6)


def test_causal_mask_right_aligned():
    assert attention.causal_mask(1, 7) is None
    m = attention.causal_mask(3, 5)
    visible = (m == 0).sum(1).tolist()
    assert visible == [3, 4, 5]
    assert np.isneginf(m[0, 3:]).all()


def test_repeat_kv_head_mapping():
    states = np.arange(2)[:, None, None] * np.ones((2, 3, 4))
    rep = attention.repeat_kv(states, 3)
    assert rep.shape == (6, 3, 4)
    assert rep[:, 0, 0].tolist() == [0, 0, 0, 1, 1, 1]        # q head i reads kv head i // 3


def test_round_to_bf16():
    torch = pytest.importorskip("torch")
    x = (np.random.default_rng(1).standard_normal(10000) * 100).astype(F32)
    x[:4] = [np.inf, -np.inf, 3.3895314e38, 1e-40]
    ours = attention.round_to_bf16(x)
    ref = torch.from_numpy(x).bfloat16().float().numpy()
    assert np.array_equal(ours, ref)


def _store(levels, key, value, **kw):
    return history.pack_history(levels, key, value, **kw)


def test_single_token_returns_its_value():
    """Empty history and tail: softmax over one key is 1 -> output = v_new."""
    levels = np.zeros((2, 8), np.int64)
    st = history.LayerHistory(levels, 4, 4, 8, 2)
    q = np.random.default_rng(2).standard_normal((4, 1, 8)).astype(F32)
    kn = np.random.default_rng(3).standard_normal((2, 1, 8)).astype(F32)
    vn = np.random.default_rng(4).standard_normal((2, 1, 8)).astype(F32)
    out = attention.reference_attention(st, q, kn, vn, 8 ** -0.5, n_q=4, n_kv=2)
    assert np.allclose(out, np.repeat(vn, 2, axis=0), atol=1e-7)


def test_equal_keys_give_mean_of_values():
    """All keys identical (lossless: one int2 group of constant K) -> uniform weights."""
    levels = np.zeros((1, 4), np.int64)
    key = np.full((1, 4, 4), 2.0, F32)
    value = np.random.default_rng(5).integers(0, 4, (1, 4, 4)).astype(F32)   # int2-exact values
    st = _store(levels, key, value, page_size=4, k_group_size=4, v_group_size=4, bit_v=2)
    kd, vd = st.dequantize()
    assert np.array_equal(kd, key)
    q = np.ones((1, 1, 4), F32)
    out = attention.reference_attention(st, q, np.full((1, 1, 4), 2.0, F32), np.zeros((1, 1, 4), F32), 0.5, 1, 1)
    expect = (vd[0].sum(0) + 0.0) / 5.0
    assert np.allclose(out[0, 0], expect, atol=1e-6)


def test_two_keys_known_weights():
    """Scores differing by ln 3 -> weights 3/4 and 1/4."""
    st = history.LayerHistory(np.zeros((1, 2), np.int64), 4, 4, 2, 2)
    st.tail_k = np.array([[[math.log(3.0), 0.0]]], F32)
    st.tail_v = np.array([[[1.0, 0.0]]], F32)
    out = attention.reference_attention(st, np.array([[[1.0, 0.0]]], F32), np.zeros((1, 1, 2), F32),
                                        np.array([[[0.0, 1.0]]], F32), 1.0, 1, 1)
    assert np.allclose(out[0, 0], [0.75, 0.25], atol=1e-6)


def test_reference_attention_concatenation_order_and_bruteforce():
    rng = np.random.default_rng(6)
    lv = rng.integers(0, 4, (2, 16))
    key = rng.standard_normal((2, 11, 16)).astype(F32)
    value = rng.standard_normal((2, 11, 16)).astype(F32)
    st = _store(lv, key, value, page_size=4, k_group_size=4, v_group_size=8, bit_v=2)
    assert st.hist_len == 8 and st.tail_len == 3
    q = rng.standard_normal((6, 1, 16)).astype(F32)
    kn = rng.standard_normal((2, 1, 16)).astype(F32)
    vn = rng.standard_normal((2, 1, 16)).astype(F32)
    kd, vd = st.dequantize()
    keys = np.concatenate([kd, key[:, 8:], kn], axis=1)
    vals = np.concatenate([vd, value[:, 8:], vn], axis=1)
    ref = brute_attention(q, np.repeat(keys, 3, 0), np.repeat(vals, 3, 0), 0.25)
    out = attention.reference_attention(st, q, kn, vn, 0.25, 6, 2)
    assert np.allclose(out, ref, atol=2e-6)
    bf = attention.reference_attention(st, q, kn, vn, 0.25, 6, 2, out_dtype="bf16")
    assert np.array_equal(bf, attention.round_to_bf16(out))


def test_history_flush_and_concatenation_axes():
    rng = np.random.default_rng(7)
    lv = rng.integers(0, 4, (3, 32))
    key = rng.standard_normal((3, 300, 32)).astype(F32)
    value = rng.standard_normal((3, 300, 32)).astype(F32)
    st = _store(lv, key, value, page_size=128, k_group_size=64, v_group_size=32, bit_v=2)
    assert (st.hist_len, st.tail_len) == (256, 44)
    table = layout.layer_table(lv)
    p0 = layout.quantize_key_page(key[:, :128], table, 64)
    p1 = layout.quantize_key_page(key[:, 128:256], table, 64)
    for t in range(3):
        assert np.array_equal(st.hist_k[t]["code"], np.concatenate([p0[t]["code"], p1[t]["code"]], 1))
        assert st.hist_k[t]["scale"].shape[2] == 4                     # groups on the innermost axis
        assert np.array_equal(st.hist_k[t]["scale"], np.concatenate([p0[t]["scale"], p1[t]["scale"]], 2))
    assert np.array_equal(st.tail_k, key[:, 256:])
    # token-by-token appends flush at the same boundaries and build the same history
    st2 = history.LayerHistory(lv, 128, 64, 32, 2)
    for t in range(300):
        st2.append(key[:, t:t + 1], value[:, t:t + 1])
    for t in range(3):
        for name in ("code", "scale", "min"):
            assert np.array_equal(st.hist_k[t][name], st2.hist_k[t][name])
    for name in ("code", "scale", "min"):
        assert np.array_equal(st.hist_v[name], st2.hist_v[name])
    assert np.array_equal(st.tail_v, st2.tail_v)
