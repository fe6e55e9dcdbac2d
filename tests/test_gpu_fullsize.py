"""Decode parity at full size: BASELINE config 2 (256 packed pages + 100 residual tokens per
sequence, 4 kv heads, GQA 7, target 2.5, batch 16 with the bench's split plan) and config 4's
shape (8 kv heads, GQA 5) with ragged contexts up to 64K tokens.

The device history of a checked sequence is exported in the reference layout (its packing is
bit-exact: the packer tests and the golden vectors pin it) and the oracle dequantises it and
attends densely in float32 (reference src/logitfill/packed/reference.py:30-56); the decode
output must meet the north-star bar, for every split pattern."""
import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import decode_into
from oracle import attention as oatt
from tests.helpers import assert_decode_close, f32, oracle_decode

pytestmark = pytest.mark.gpu


def _np_history(layer, b):
    hk, hv = layer.export_reference(b)
    return ({t: {k: v.cpu().numpy() for k, v in d.items()} for t, d in hk.items()},
            {k: v.cpu().numpy() for k, v in hv.items()})


def _build(gpu, B, n_q, n_kv, pages, resid, target, seed):
    d = synth.make_layer(B, n_q, n_kv, 128, max(pages) * 128 + 128, target, seed=seed, device=gpu)
    mgr = PackedKVManager([d.levels], n_q, n_kv, 128, 128, 128, 128, 2, gpu, batch_size=B,
                          capacity_tokens=max(pages) * 128)
    st = mgr.layers[0]
    st.fill_pages(d.key, d.value, pages)
    rk = torch.stack([d.key[b, :, pages[b] * 128:pages[b] * 128 + 127] for b in range(B)])
    rv = torch.stack([d.value[b, :, pages[b] * 128:pages[b] * 128 + 127] for b in range(B)])
    st.set_tail(rk, rv, resid)
    return d, mgr


def _oracle(d, mgr, b, n_q, n_kv, scaling):
    st = mgr.layers[0]
    hk, hv = _np_history(st, b)
    tl = st.tail_lens[b]
    tk, tv = st.tail_buffers()
    store = oatt.ExportedHistory(d.levels, hk, hv, st.hist_lens[b], f32(tk[b, :, :tl]), f32(tv[b, :, :tl]), 128, 128, 2)
    return oracle_decode(store, f32(d.query[b]), f32(d.key_new[b]), f32(d.value_new[b]), scaling, n_q, n_kv)


def _decode(d, mgr, gpu, scaling, pages_per_split=None, out_dtype=None):
    q = d.query
    out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=gpu)
    decode_into(mgr, 0, q, d.key_new, d.value_new, scaling, out, kernel=_native.KERNEL_MFMA,
                pages_per_split=pages_per_split)
    torch.cuda.synchronize()
    return out


def test_headline_shape_full_size(gpu):
    """c2: 16 sequences x (256 pages + 100 residual + the new token), the bench's plan (the
    paired plan on 256 CUs: every sequence's 4 first items of 36 pages listed before all
    second items of 29, 29, 29 and 25 pages + the residual, partials in per-sequence slots);
    the first, a middle and the last sequence checked."""
    B, n_q, n_kv = 16, 28, 4
    d, mgr = _build(gpu, B, n_q, n_kv, [256] * B, [100] * B, 2.5, seed=11)
    scaling = 128 ** -0.5
    out = _decode(d, mgr, gpu, scaling)
    plan = mgr.layers[0].decode_plan
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert plan.pages_per_split == ("paired", 36, 0) and plan.n_work == 128
    for b in (0, 9, 15):
        print(f"c2 full size: sequence {b}", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))


def test_headline_shape_every_split_meets_the_bar(gpu):
    """The same c2 layer with 8-, 33- (the bench's) and 300-page items (one item per sequence):
    every split pattern meets the bar against the oracle.  A long item is where the Value
    product's offset cancellation (p * (4 + code) against the per-token constant) would build
    up; the kernel folds it every 64 pages."""
    B, n_q, n_kv = 16, 28, 4
    d, mgr = _build(gpu, B, n_q, n_kv, [256] * B, [100] * B, 2.5, seed=12)
    scaling = 128 ** -0.5
    outs = {s: _decode(d, mgr, gpu, scaling, pages_per_split=s) for s in (8, 33, 300)}
    for b in (3, 15):
        ref = _oracle(d, mgr, b, n_q, n_kv, scaling)
        for s, out in outs.items():
            print(f"c2 full size: sequence {b}, {s}-page items", flush=True)
            assert_decode_close(out[b], ref)


def test_config4_longest_contexts(gpu):
    """c4's shape (40 q / 8 kv heads, target 2.5) with ragged contexts U[4K, 64K] (seeded) plus
    one sequence at 64K: the two longest sequences and the shortest are checked."""
    B, n_q, n_kv = 6, 40, 8
    pages, resid = synth.ragged_lengths(B - 1, seed=4)
    pages = pages + [511]          # 65 408 history tokens
    resid = resid + [127]
    d, mgr = _build(gpu, B, n_q, n_kv, pages, resid, 2.5, seed=13)
    scaling = 128 ** -0.5
    out = _decode(d, mgr, gpu, scaling)
    order = np.argsort(pages)
    for b in (int(order[-1]), int(order[-2]), int(order[0])):
        print(f"c4 shape: sequence {b}, {pages[b]} pages + {resid[b]}", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))


def test_config4_full_batch_bench_plan(gpu):
    """c4 at its own workload: 32 sequences with the bench's seeded ragged contexts U[4K, 64K]
    (``synth.ragged_lengths(32, seed=4)``, residuals 1-127), 40 q / 8 kv heads, target 2.5,
    decoded with the automatic split the bench times (the planner's size, sequences dispatched
    by decreasing item size).  Checked against the oracle: the first and the last sequence in
    that dispatch order, the longest, the shortest and a middle one."""
    from logitfill_amd.packed.reference import plan_work, residual_pages

    B, n_q, n_kv = 32, 40, 8
    pages, resid = synth.ragged_lengths(B, seed=4)
    d, mgr = _build(gpu, B, n_q, n_kv, pages, resid, 2.5, seed=14)
    scaling = 128 ** -0.5
    q = d.query
    out = torch.empty(q.shape, dtype=q.dtype, device=gpu)
    decode_into(mgr, 0, q, d.key_new, d.value_new, scaling, out)   # the bench's call: auto kernel and split
    torch.cuda.synchronize()
    plan = mgr.layers[0].decode_plan
    work = plan.work.cpu().numpy().reshape(-1, 4)
    assert plan.n_work == work.shape[0] and plan.n_work > B        # split-K over ragged page counts
    size = plan.pages_per_split
    sizes = [size] * B if isinstance(size, int) else list(size)
    want, _ = plan_work(pages, sizes, residual_pages(resid))
    assert np.array_equal(work.reshape(-1), np.asarray(want))      # the plan the bench dispatches
    dispatch = list(dict.fromkeys(int(b) for b in work[:, 0]))     # sequences in dispatch order
    order = np.argsort(pages, kind="stable")
    picks = dict.fromkeys([dispatch[0], dispatch[-1], int(order[-1]), int(order[0]), int(order[B // 2])])
    for b in picks:
        print(f"c4 batch 32: sequence {b}, {pages[b]} pages + {resid[b]}, "
              f"{int((work[:, 0] == b).sum())} items", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))


def test_single_64k_sequence_paired_plan(gpu):
    """One sequence at the largest BASELINE context (512 pages = 64K tokens + a 100-token
    residual), 40 q / 8 kv heads (c4's head shape): the planner pairs its items on 256 CUs --
    32 first items of 9 pages listed before 32 second items sharing the rest, partials in the
    sequence's 64 slots -- and the output meets the bar against the oracle."""
    B, n_q, n_kv = 1, 40, 8
    d, mgr = _build(gpu, B, n_q, n_kv, [512], [100], 2.5, seed=17)
    scaling = 128 ** -0.5
    out = _decode(d, mgr, gpu, scaling)
    plan = mgr.layers[0].decode_plan
    if torch.cuda.get_device_properties(gpu).multi_processor_count == 256:
        assert plan.pages_per_split == ("paired", 9, 0) and plan.n_work == 64
    print("single 64K sequence, paired plan", flush=True)
    assert_decode_close(out[0], _oracle(d, mgr, 0, n_q, n_kv, scaling))


@pytest.mark.parametrize("kernel", [_native.KERNEL_MFMA, _native.KERNEL_VALU])
def test_target_4_tier_mix(gpu, kernel):
    """c2's head shape at target 4.0 (Key 6.0 bits: up to 34 int8 and 13 fp16 channels per kv
    head, the widest tier mix BASELINE names), 4 sequences x 64 pages + a 100-token residual,
    with both decode kernels: every sequence meets the bar against the oracle."""
    B, n_q, n_kv = 4, 28, 4
    d, mgr = _build(gpu, B, n_q, n_kv, [64] * B, [100] * B, 4.0, seed=19)
    assert mgr.layers[0].widths[3] > 8 and mgr.layers[0].words[2] >= 8
    scaling = 128 ** -0.5
    q = d.query
    out = torch.empty(q.shape, dtype=q.dtype, device=gpu)
    decode_into(mgr, 0, q, d.key_new, d.value_new, scaling, out, kernel=kernel)
    torch.cuda.synchronize()
    for b in range(B):
        print(f"target 4.0: kernel {kernel}, sequence {b}", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))
