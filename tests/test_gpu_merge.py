"""The split-K plan and merge of the packed decode (the reduce kernel over the splits' softmax
partials) against the oracle (reference src/logitfill/packed/reference.py:30-56 over
[history ; tail ; new]): forced split sizes that give every sequence 1 .. 12 items, ragged
item counts, the dispatch-order split (two item sizes), and layers decoded back to back on one
stream whose partials reuse the same workspace addresses."""
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import age_split, choose_pages_per_split, decode_into, residual_pages
from oracle import attention as oatt
from tests.helpers import assert_decode_close, f32

pytestmark = pytest.mark.gpu

D = 128


def _check_against_oracle(st, d, out, seqs, levels, n_q, n_kv, tail):
    tk, tv = st.tail_buffers()
    for b in seqs:
        hk, hv = st.export_reference(b)
        hk = {t: {k: v.cpu().numpy() for k, v in x.items()} for t, x in hk.items()} if hk is not None else None
        hv = {k: v.cpu().numpy() for k, v in hv.items()} if hv is not None else None
        store = oatt.ExportedHistory(levels, hk, hv, st.hist_lens[b], f32(tk[b, :, :tail]), f32(tv[b, :, :tail]),
                                     128, 128, 2)
        ref = oatt.reference_attention(store, f32(d.query[b])[:, None, :], f32(d.key_new[b])[:, None, :],
                                       f32(d.value_new[b])[:, None, :], D ** -0.5, n_q, n_kv)[:, 0, :]
        print(f"merge: sequence {b}", flush=True)
        assert_decode_close(out[b], ref, out_dtype="fp32")


def _layer(gpu, B, n_q, n_kv, pages, tail, seed):
    d = synth.make_layer(B, n_q, n_kv, D, pages * 128 + 128, 2.5, seed=seed, device=gpu)
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B,
                          capacity_tokens=max(pages, 1) * 128)
    st = mgr.layers[0]
    if pages:
        st.fill_pages(d.key, d.value, [pages] * B)
    st.set_tail(d.key[:, :, pages * 128:pages * 128 + 127], d.value[:, :, pages * 128:pages * 128 + 127], [tail] * B)
    return d, mgr, st


@pytest.mark.parametrize("pps", [1, 3, None])
def test_split_sizes_merge_to_the_oracle(gpu, pps):
    """Sequences split into 1-page items (12 + the residual's), 3-page items and the planner's
    size, the matrix-core kernel; two calls in a row on the same workspace."""
    B, n_q, n_kv, pages, tail = 4, 28, 4, 12, 45
    d, mgr, st = _layer(gpu, B, n_q, n_kv, pages, tail, seed=71)
    out = torch.empty(B, n_q, D, dtype=torch.float32, device=gpu)
    for _ in range(2):
        decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=_native.KERNEL_MFMA,
                    pages_per_split=pps)
        torch.cuda.synchronize()
    _check_against_oracle(st, d, out, range(B), d.levels, n_q, n_kv, tail)


def test_ragged_items_divisible_by_the_batch(gpu):
    """Sequences of 9 and 1 pages at 3 pages per item: 4 + 2 items, a total the batch divides
    although the sequences' counts differ, so only the plan's own (first, count) per sequence
    merges the right items."""
    B, n_q, n_kv, tail = 2, 28, 4, 30
    d = synth.make_layer(B, n_q, n_kv, D, 10 * 128, 2.5, seed=73, device=gpu)
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B, capacity_tokens=9 * 128)
    st = mgr.layers[0]
    st.fill_pages(d.key, d.value, [9, 1])
    rk = torch.stack([d.key[b, :, p * 128:p * 128 + 127] for b, p in enumerate([9, 1])])
    rv = torch.stack([d.value[b, :, p * 128:p * 128 + 127] for b, p in enumerate([9, 1])])
    st.set_tail(rk, rv, [tail] * B)
    out = torch.empty(B, n_q, D, dtype=torch.float32, device=gpu)
    decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=_native.KERNEL_MFMA, pages_per_split=3)
    torch.cuda.synchronize()
    plan = st.decode_plan
    seq = plan.seq_work.cpu().tolist()
    assert plan.n_work % B == 0 and seq[1] != plan.n_work // B
    _check_against_oracle(st, d, out, range(B), d.levels, n_q, n_kv, tail)


def test_back_to_back_layers_share_the_workspace(gpu):
    """Six layers decoded back to back on one stream with no synchronisation between them: each
    layer's splits write their partials to the same workspace addresses as the layer before
    (on whatever XCD they land) and each layer's merge must read its own layer's values."""
    B, n_q, n_kv, pages, tail, n_layers = 6, 28, 4, 9, 30, 6
    ds = [synth.make_layer(B, n_q, n_kv, D, pages * 128 + 128, 2.5, seed=80 + l, device=gpu) for l in range(n_layers)]
    mgr = PackedKVManager([d.levels for d in ds], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B,
                          capacity_tokens=pages * 128)
    for l, d in enumerate(ds):
        st = mgr.layers[l]
        st.fill_pages(d.key, d.value, [pages] * B)
        st.set_tail(d.key[:, :, pages * 128:pages * 128 + 127], d.value[:, :, pages * 128:pages * 128 + 127], [tail] * B)
    outs = [torch.empty(B, n_q, D, dtype=torch.float32, device=gpu) for _ in range(n_layers)]
    torch.cuda.synchronize()
    for l, d in enumerate(ds):
        decode_into(mgr, l, d.query, d.key_new, d.value_new, D ** -0.5, outs[l], kernel=_native.KERNEL_MFMA,
                    pages_per_split=2)
    torch.cuda.synchronize()
    for l, d in enumerate(ds):
        print(f"merge: layer {l}", flush=True)
        _check_against_oracle(mgr.layers[l], d, outs[l], [0, B - 1], d.levels, n_q, n_kv, tail)


@pytest.mark.parametrize("B,n_q,n_kv,pages,tail", [(8, 12, 2, 200, 50), (4, 28, 4, 256, 20)])
def test_dispatch_order_splits_match_the_oracle(gpu, B, n_q, n_kv, pages, tail):
    """Batches of equal sequences whose plan fills one round: the planner's choice (on 256 CUs
    the paired plan, first items listed first, partials in per-sequence slots) and the
    two-size dispatch-order split (the first sequences in fewer, larger items: two item sizes,
    the larger first) both match the oracle."""
    d, mgr, st = _layer(gpu, B, n_q, n_kv, pages, tail, seed=74 + B)
    res = residual_pages([tail])
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    out = torch.empty(B, n_q, D, dtype=torch.float32, device=gpu)
    decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=_native.KERNEL_MFMA)
    torch.cuda.synchronize()
    choice = st.decode_plan.pages_per_split
    if cus == 256:
        assert isinstance(choice, tuple) and choice[0] == "paired"
        assert st.decode_plan.n_work * n_kv == 2 * cus
    print(f"dispatch-order: planner's choice {choice}", flush=True)
    _check_against_oracle(st, d, out, [0, B // 2, B - 1], d.levels, n_q, n_kv, tail)
    size = choose_pages_per_split([pages] * B, n_kv, res, gpu)
    sizes = tuple(age_split([pages] * B, n_kv, res, size, cus))
    assert len(set(sizes)) == 2 and sizes[0] > sizes[-1]
    decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=_native.KERNEL_MFMA,
                pages_per_split=sizes)
    torch.cuda.synchronize()
    seq = st.decode_plan.seq_work.cpu().tolist()
    assert [seq[2 * b + 1] for b in range(B)] == [-(-(pages + res) // z) for z in sizes]
    print("dispatch-order: two-size split", flush=True)
    _check_against_oracle(st, d, out, [0, B - 1], d.levels, n_q, n_kv, tail)


@pytest.mark.parametrize("kernel,pps", [(_native.KERNEL_MFMA, None), (_native.KERNEL_MFMA, 1),
                                        (_native.KERNEL_VALU, 3)])
def test_plan_in_the_kernel_arguments_matches_the_device_plan(gpu, kernel, pps):
    """The host copies of the plan (lf_decode_args.work_host / seq_work_host) put the work
    records and the sequences' item ranges into the kernels' argument blocks; without them the
    kernels read the device plan.  Same outputs bit for bit, and against the oracle.  With
    1-page items 8 sequences x 15 items (120 <= LF_INLINE_WORK = 208) stay inline; 10
    sequences x 23 items (230) read their work records from the device list while their
    sequence ranges stay inline."""
    n_q, n_kv, tail = 28, 4, 45
    for B, pages in ((8, 12), (10, 20)):
        if pps != 1 and pages == 20:
            continue
        d, mgr, st = _layer(gpu, B, n_q, n_kv, pages, tail, seed=73 + pages)
        outs = []
        for inline in (True, False):
            if not inline:  # the same cached argument block without the host copies
                a = st.__dict__["_lf_decode_args"][1]
                a.work_host, a.seq_work_host = 0, 0
            out = torch.empty(B, n_q, D, dtype=torch.float32, device=gpu)
            decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=kernel, pages_per_split=pps)
            torch.cuda.synchronize()
            if inline:
                assert st.__dict__["_lf_decode_args"][1].work_host != 0
            outs.append(out)
        if pps == 1:
            assert (st.decode_plan.n_work > 208) == (pages == 20)
        print(f"inline plan: B {B} pages {pages} pps {pps} kernel {kernel} items {st.decode_plan.n_work}", flush=True)
        assert torch.equal(outs[0], outs[1])
        _check_against_oracle(st, d, outs[0], (0, B - 1), d.levels, n_q, n_kv, tail)


@pytest.mark.parametrize("kernel,choice", [(_native.KERNEL_MFMA, ("paired", 7, 0)),
                                           (_native.KERNEL_VALU, ("paired", 7, 0)),
                                           (_native.KERNEL_MFMA, ("paired", 9, 2)),
                                           (_native.KERNEL_VALU, ("paired", 9, 2))])
def test_paired_plan_merges_to_the_oracle(gpu, kernel, choice):
    """The paired plans (items listed first-items-first, each partial in its sequence's slot
    range through the kind field): 4 sequences x 200 pages, 4 kv heads, 16 first items per
    sequence on 256 CUs, then 16 second items sharing the rest with the residual on the last,
    or 2-page items and a residual-only item; both kernels against the oracle, and the same
    outputs as a contiguous plan."""
    if torch.cuda.get_device_properties(gpu).multi_processor_count != 256:
        pytest.skip("the plan below is sized for 256 CUs")
    B, n_q, n_kv, pages, tail = 4, 28, 4, 200, 45
    d, mgr, st = _layer(gpu, B, n_q, n_kv, pages, tail, seed=79)
    res = residual_pages([tail])
    outs = []
    for pps in (choice, 25):
        out = torch.empty(B, n_q, D, dtype=torch.float32, device=gpu)
        decode_into(mgr, 0, d.query, d.key_new, d.value_new, D ** -0.5, out, kernel=kernel, pages_per_split=pps)
        torch.cuda.synchronize()
        outs.append(out)
    print(f"paired plan: kernel {kernel} residual {res}", flush=True)
    _check_against_oracle(st, d, outs[0], range(B), d.levels, n_q, n_kv, tail)
    torch.testing.assert_close(outs[0], outs[1], rtol=2e-3, atol=2e-4)
