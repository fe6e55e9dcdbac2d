"""Deferred page flushes and the multi-layer page compress (lf_pack_pages_multi).

The reference packs a layer's full residual page inside that layer's commit
(src/logitfill/packed/cache.py:54-81).  A deferring manager leaves the full page in
the residual buffer and packs every layer's pages in one launch at the end of the
step; the packed history must be bit-identical to the eager one (and to the oracle
store), and any reader of a layer's history must see the page packed."""
import ctypes

import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import packed_attention
from tests.helpers import assert_decode_close, assert_history_equal, f32, oracle_store

pytestmark = pytest.mark.gpu


def test_deferred_flush_matches_eager_and_oracle(gpu):
    """3 layers of different tier widths, batch 2 with ragged prefills (120, 60 tokens), then
    150 one-token steps committing every layer; the deferring manager flushes once per step."""
    n_kv, D, L, steps = 2, 128, 3, 150
    lens = [120, 60]
    data = [[synth.make_layer(1, 4, n_kv, D, 300, 2.5 + 0.5 * i, seed=40 + 10 * i + b) for b in range(2)]
            for i in range(L)]
    levels = [data[i][0].levels for i in range(L)]
    eager = PackedKVManager(levels, 4, n_kv, D, 128, 128, 128, 2, gpu, batch_size=2)
    lazy = PackedKVManager(levels, 4, n_kv, D, 128, 128, 128, 2, gpu, batch_size=2, defer_flush=True)
    for i in range(L):
        k0 = torch.zeros(2, n_kv, max(lens), D, dtype=torch.bfloat16)
        v0 = torch.zeros_like(k0)
        for b in range(2):
            k0[b, :, :lens[b]] = data[i][b].key[0, :, :lens[b]]
            v0[b, :, :lens[b]] = data[i][b].value[0, :, :lens[b]]
        for m in (eager, lazy):
            m.commit(i, k0.to(gpu), v0.to(gpu), lengths=lens)
    flushed_steps = 0
    for t in range(steps):
        for i in range(L):
            kt = torch.stack([data[i][b].key[0, :, lens[b] + t] for b in range(2)])[:, :, None].to(gpu)
            vt = torch.stack([data[i][b].value[0, :, lens[b] + t] for b in range(2)])[:, :, None].to(gpu)
            eager.commit(i, kt, vt)
            lazy.commit(i, kt, vt)
        if any(layer.pending for layer in lazy.layers):
            # every layer fills its page on the same token
            assert all(layer.pending == lazy.layers[0].pending for layer in lazy.layers)
            assert all(layer.tail_lens[b] == 128 for layer in lazy.layers for b, _ in layer.pending)
            flushed_steps += 1
        lazy.flush_pending()
        assert not any(layer.pending for layer in lazy.layers)
        assert [lay.hist_lens for lay in lazy.layers] == [lay.hist_lens for lay in eager.layers]
        assert [lay.tail_lens for lay in lazy.layers] == [lay.tail_lens for lay in eager.layers]
    assert flushed_steps >= 2
    torch.cuda.synchronize()
    for i in range(L):
        for b in range(2):
            n = lens[b] + steps
            store = oracle_store(levels[i], f32(data[i][b].key[0, :, :n]), f32(data[i][b].value[0, :, :n]))
            assert_history_equal(lazy.layers[i], b, store)
            assert_history_equal(eager.layers[i], b, store)


def test_pending_page_is_packed_before_attention(gpu):
    """A page completed by a deferred commit is packed by the next reader: packed attention
    on that layer before flush_pending gives exactly the eager manager's output."""
    n_kv, D = 4, 128
    d = synth.make_layer(1, 28, n_kv, D, 256, 2.5, seed=3)
    eager = PackedKVManager([d.levels], 28, n_kv, D, 128, 128, 128, 2, gpu)
    lazy = PackedKVManager([d.levels], 28, n_kv, D, 128, 128, 128, 2, gpu, defer_flush=True)
    k, v = d.key.to(gpu), d.value.to(gpu)
    for m in (eager, lazy):
        m.commit(0, k[:, :, :255], v[:, :, :255])
        m.commit(0, k[:, :, 255:], v[:, :, 255:])     # fills page 1
    assert lazy.layers[0].pending == [(0, 1)]
    q = d.query[:, :, None].to(gpu)
    kn = torch.randn(1, n_kv, 1, D, generator=torch.Generator().manual_seed(1)).bfloat16().to(gpu)
    vn = torch.randn(1, n_kv, 1, D, generator=torch.Generator().manual_seed(2)).bfloat16().to(gpu)
    out_e = packed_attention(eager, 0, q[:, :, :1], kn, vn, D ** -0.5)
    out_l = packed_attention(lazy, 0, q[:, :, :1], kn, vn, D ** -0.5)
    assert lazy.layers[0].pending == []
    assert torch.equal(out_e, out_l)
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]))
    assert_history_equal(lazy.layers[0], 0, store)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_pack_pages_multi_matches_per_layer(gpu, dtype):
    """Direct lf_pack_pages_multi call: 4 layers with their own tier tables and page sources
    (strided views), several sequences and destination pages per layer, one launch; equal to
    one lf_pack_pages launch per layer."""
    n_kv, D, B, L = 4, 128, 3, 4
    lib = _native.load()
    srcs, one, multi = [], [], []
    for i in range(L):
        d = synth.make_layer(B, 28, n_kv, D, 256, 2.5 + 0.5 * i, seed=70 + i, dtype=dtype)
        big_k = torch.zeros(B, n_kv, 384, D, dtype=dtype)
        big_v = torch.zeros_like(big_k)
        big_k[:, :, 64:320] = d.key
        big_v[:, :, 64:320] = d.value
        srcs.append((big_k.to(gpu)[:, :, 64:320], big_v.to(gpu)[:, :, 64:320]))
        for lst in (one, multi):
            lst.append(PackedKVManager([d.levels], 28, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B,
                                       capacity_tokens=512))
    jobs = [(b, 128 * p, (p + b) % 4) for b in range(B) for p in range(2)]   # (b, src token, dst page)
    stream = _native.current_stream_ptr(gpu)
    jd = torch.tensor(jobs, dtype=torch.int32).to(gpu)
    for i, (k, v) in enumerate(srcs):
        st = lib.lf_pack_pages(one[i].layers[0].layer_struct(), k.data_ptr(), v.data_ptr(), _native.dtype_code(dtype),
                               k.stride(0), k.stride(1), k.stride(2), jd.data_ptr(), len(jobs), stream)
        _native.check(st, "lf_pack_pages")
    structs = (_native.PackedLayer * L)(*[m.layers[0].layer_struct() for m in multi])
    ps = (_native.PackSource * L)(*[_native.PackSource(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                                                       k.stride(2)) for k, v in srcs])
    dev_structs = torch.frombuffer(bytearray(structs), dtype=torch.uint8).to(gpu)
    dev_ps = torch.frombuffer(bytearray(ps), dtype=torch.uint8).to(gpu)
    mjobs = torch.tensor([(i, *j) for i in range(L) for j in jobs], dtype=torch.int32).to(gpu)
    st = lib.lf_pack_pages_multi(dev_structs.data_ptr(), structs, dev_ps.data_ptr(), ps, L, _native.dtype_code(dtype),
                                 mjobs.data_ptr(), mjobs.shape[0], stream)
    _native.check(st, "lf_pack_pages_multi")
    torch.cuda.synchronize()
    for i in range(L):
        a, b = one[i].layers[0]._s, multi[i].layers[0]._s
        for name in ("k_code", "k_scale", "k_min"):
            for t in range(3):
                assert torch.equal(a[name][t].view(torch.uint8), b[name][t].view(torch.uint8)), (i, name, t)
        for name in ("k_value16", "v_code", "v_scale", "v_min"):
            assert torch.equal(a[name].view(torch.uint8), b[name].view(torch.uint8)), (i, name)
    # written pages hold data (the comparison above is not between two untouched buffers)
    assert int((multi[0].layers[0]._s["v_code"] != 0).sum()) > 0


def test_pack_pages_multi_rejects_other_shapes(gpu):
    """A layer outside the fast shape (head_dim 64) is refused before launch; the manager then
    flushes layer by layer."""
    lib = _native.load()
    d = synth.make_layer(1, 4, 2, 64, 64, 2.5, seed=1)
    m = PackedKVManager([d.levels, d.levels], 4, 2, 64, 64, 64, 64, 2, gpu, defer_flush=True)
    structs = (_native.PackedLayer * 2)(*[lay.layer_struct() for lay in m.layers])
    k = torch.zeros(1, 2, 64, 64, dtype=torch.bfloat16, device=gpu)
    ps = (_native.PackSource * 2)(*[_native.PackSource(k.data_ptr(), k.data_ptr(), k.stride(0), k.stride(1),
                                                       k.stride(2))] * 2)
    jobs = torch.zeros(1, 4, dtype=torch.int32, device=gpu)
    dummy = ctypes.c_void_p(k.data_ptr())
    st = lib.lf_pack_pages_multi(dummy, structs, dummy, ps, 2, _native.LF_BF16, jobs.data_ptr(), 1,
                                 _native.current_stream_ptr(gpu))
    assert st == _native.LF_E_UNSUPPORTED
    kk, vv = d.key.to(gpu), d.value.to(gpu)
    for i in range(2):
        m.commit(i, kk, vv)
    assert all(lay.pending == [(0, 0)] for lay in m.layers)
    m.flush_pending()
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]), 64, 64, 64, 2)
    for lay in m.layers:
        assert_history_equal(lay, 0, store)
    assert np.all([lay.pending == [] for lay in m.layers])


@pytest.mark.parametrize("defer", [False, True])
def test_device_append_path_matches_oracle(gpu, defer):
    """One contiguous token per sequence per step -- the model's decode commit -- goes through
    lf_append_token (rows written at the device-side residual lengths, which it advances; no
    upload).  Batch 3 with ragged prefills, 140 steps across page flushes: every sequence's
    history and residual equal the oracle store's, the device lengths equal the host's, and a
    decode at the end matches the oracle (reference cache.py:48-90, reference.py:30-56)."""
    from logitfill_amd.packed.reference import packed_attention
    from oracle import attention as oatt

    n_q, n_kv, D, B, steps = 4, 2, 128, 3, 140
    lens = [120, 7, 64]
    ds = [synth.make_layer(1, n_q, n_kv, D, 300, 2.5, seed=60 + b) for b in range(B)]
    levels = ds[0].levels
    m = PackedKVManager([levels], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B, defer_flush=defer)
    k0 = torch.zeros(B, n_kv, max(lens), D, dtype=torch.bfloat16)
    v0 = torch.zeros_like(k0)
    for b in range(B):
        k0[b, :, :lens[b]] = ds[b].key[0, :, :lens[b]]
        v0[b, :, :lens[b]] = ds[b].value[0, :, :lens[b]]
    m.commit(0, k0.to(gpu), v0.to(gpu), lengths=lens)
    keys = torch.stack([d.key[0] for d in ds])       # [B, n_kv, 300, D]
    values = torch.stack([d.value[0] for d in ds])
    appended = 0
    for s in range(steps):
        kt = torch.stack([keys[b, :, lens[b] + s] for b in range(B)])[:, :, None].contiguous().to(gpu)
        vt = torch.stack([values[b, :, lens[b] + s] for b in range(B)])[:, :, None].contiguous().to(gpu)
        before = list(m.layers[0].tail_lens)
        m.commit(0, kt, vt)
        if defer:
            m.flush_pending()
        appended += int(max(before) + 1 < 128 and not m.layers[0].pending)
    layer = m.layers[0]
    assert appended > 100  # most steps took the device append path
    assert layer.tail_len_device().cpu().tolist() == layer.tail_lens
    for b in range(B):
        n = lens[b] + steps
        store = oracle_store(levels, f32(keys[b, :, :n]), f32(values[b, :, :n]))
        assert_history_equal(layer, b, store)
    q = torch.randn(B, n_q, 1, D, generator=torch.Generator().manual_seed(3)).bfloat16().to(gpu) * D ** -0.5
    kn = torch.randn(B, n_kv, 1, D, generator=torch.Generator().manual_seed(4)).bfloat16().to(gpu)
    vn = torch.randn(B, n_kv, 1, D, generator=torch.Generator().manual_seed(5)).bfloat16().to(gpu)
    out = packed_attention(m, 0, q, kn, vn, D ** -0.5)
    for b in range(B):
        n = lens[b] + steps
        store = oracle_store(levels, f32(keys[b, :, :n]), f32(values[b, :, :n]))
        ref = oatt.reference_attention(store, f32(q[b]), f32(kn[b]), f32(vn[b]), D ** -0.5, n_q, n_kv)
        assert_decode_close(out[b, :, 0], ref[:, 0])


def test_decode_step_replays_from_a_hip_graph(gpu):
    """A decode step -- every layer's packed_attention then a one-token commit through
    lf_append_token -- captured once in a HIP graph and replayed: each replay appends one more
    token (positions live on the device) and its outputs equal, bit for bit, those of an eager
    twin manager stepped with the same inputs; the program's own eager work and
    synchronisations run between the replays."""
    n_q, n_kv, D, B, L = 8, 2, 128, 2, 3
    ds = [synth.make_layer(B, n_q, n_kv, D, 5 * 128 + 20, 2.5, seed=90 + i) for i in range(L)]
    levels = [d.levels for d in ds]
    mgrs = [PackedKVManager(levels, n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B) for _ in range(2)]
    for m in mgrs:
        for i, d in enumerate(ds):
            m.commit(i, d.key.to(gpu), d.value.to(gpu))
    ins = [(d.query[:, :, None].contiguous().to(gpu), d.key_new[:, :, None].contiguous().to(gpu),
            d.value_new[:, :, None].contiguous().to(gpu)) for d in ds]

    def step(m):
        outs = []
        for i, (q, kn, vn) in enumerate(ins):
            outs.append(packed_attention(m, i, q, kn, vn, D ** -0.5))
            m.commit(i, kn, vn)
        return outs

    eager, graphed = mgrs
    step(graphed)          # warm-up outside capture: plans, workspace, device lengths
    step(eager)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            captured = step(graphed)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for r in range(5):
        g.replay()
        want = step(eager)
        torch.cuda.synchronize()
        for i in range(L):
            assert torch.equal(captured[i], want[i]), (r, i)
        tl = graphed.layers[0].tail_len_device().cpu().tolist()
        assert tl == eager.layers[0].tail_lens, (r, tl)
