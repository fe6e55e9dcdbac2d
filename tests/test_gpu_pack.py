"""GPU parity of the page-compress kernel: bit-exact codes, scales, mins and fp16
values against the oracle packer (reference src/logitfill/packed/layout.py:71-129,
history axes of cache.py:64-81) on the same seeded inputs."""
import numpy as np
import pytest
import torch

from logitfill_amd import synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed import layout as pl
from oracle import layout as ol
from tests.helpers import assert_history_equal, f32, oracle_store

pytestmark = pytest.mark.gpu


def make_manager(levels, n_q, n_kv, D, dev, page=128, kg=128, vg=128, bit_v=2, batch=1):
    return PackedKVManager([levels], n_q, n_kv, D, page, kg, vg, bit_v, dev, batch_size=batch)


def test_config0_pack_bit_exact(gpu):
    """8 full pages, 4 kv heads, D 128, target 2.5."""
    d = synth.make_layer(1, 28, 4, 128, 1024, 2.5, seed=0)
    mgr = make_manager(d.levels, 28, 4, 128, gpu)
    mgr.commit(0, d.key.to(gpu), d.value.to(gpu))
    torch.cuda.synchronize()
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]))
    assert_history_equal(mgr.layers[0], 0, store)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_input_dtypes_bit_exact(gpu, dtype):
    d = synth.make_layer(1, 8, 2, 128, 256, 3.0, seed=5, dtype=dtype)
    mgr = make_manager(d.levels, 8, 2, 128, gpu)
    mgr.commit(0, d.key.to(gpu), d.value.to(gpu))
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]))
    assert_history_equal(mgr.layers[0], 0, store)


def test_reference_kernel_test_shape(gpu):
    """The reference's CUDA test shape (tests/test_logitfill_offline.py:198-213): D 64,
    page = groups = 64, all four tiers, one page of float32 randn."""
    g = torch.Generator().manual_seed(0)
    levels = torch.randint(0, 4, (1, 64), generator=g)
    key = torch.randn(1, 1, 64, 64, generator=g)
    value = torch.randn(1, 1, 64, 64, generator=g)
    mgr = PackedKVManager([levels], 1, 1, 64, 64, 64, 64, 2, gpu)
    mgr.commit(0, key.to(gpu), value.to(gpu))
    store = oracle_store(levels.numpy(), key[0].numpy(), value[0].numpy(), 64, 64, 64, 2)
    assert_history_equal(mgr.layers[0], 0, store)


@pytest.mark.parametrize("kg,vg,bit_v", [(64, 128, 2), (32, 64, 2), (128, 32, 4), (128, 16, 8), (128, 128, 16)])
def test_group_and_value_width_variants(gpu, kg, vg, bit_v):
    d = synth.make_layer(1, 4, 2, 128, 384, 3.0, seed=kg + vg + bit_v)
    mgr = make_manager(d.levels, 4, 2, 128, gpu, kg=kg, vg=vg, bit_v=bit_v)
    mgr.commit(0, d.key.to(gpu), d.value.to(gpu))
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]), 128, kg, vg, bit_v)
    assert_history_equal(mgr.layers[0], 0, store)


def test_edge_values_bit_exact(gpu):
    """Constant groups (s clamps to 1e-5), huge ranges (fp16 inf scale), exact .5 ties,
    tiny and subnormal-range values, signed zeros, fp16-overflowing fp16-tier values."""
    D, T = 64, 128
    levels = np.tile(np.array([0, 1, 2, 3]), 16)[None].repeat(2, 0)
    key = torch.randn(1, 2, T, D) * 3
    key[0, 0, :, 0] = 7.0                                   # constant int2 group
    key[0, 0, :, 1] = torch.linspace(-3e5, 3e5, T)          # int4, range > fp16 max * 15
    key[0, 0, :, 4] = torch.tensor([0.0, 0.5, 1.5, 2.5, 3.0] * 25 + [0.0, 0.0, 3.0])   # int2 ties
    key[0, 1, :, 0] = torch.randn(T) * 1e-30                # tiny (fp16 min -> 0/subnormal)
    key[0, 1, :, 3] = torch.randn(T) * 1e5                  # fp16 tier overflows to +-inf
    key[0, 1, :, 7] = -0.0
    key = key.bfloat16()
    value = (torch.randn(1, 2, T, D) * torch.logspace(-6, 6, D)).bfloat16()
    value[0, 0, 3] = 1.0
    mgr = PackedKVManager([levels], 2, 2, D, 128, 128, 64, 2, gpu)
    mgr.commit(0, key.to(gpu), value.to(gpu))
    store = oracle_store(levels, f32(key[0]), f32(value[0]), 128, 128, 64, 2)
    assert_history_equal(mgr.layers[0], 0, store)


def test_edge_values_bit_exact_128(gpu):
    """The same edge cases at the common shape (D 128, page = groups = 128, int2 Values: the
    1024-thread page-compress path), plus a Value row with a huge range."""
    D, T = 128, 256
    levels = np.tile(np.array([0, 1, 2, 3, 0, 0, 1, 0]), 16)[None].repeat(2, 0)
    key = torch.randn(1, 2, T, D) * 3
    key[0, 0, :128, 0] = 7.0                                  # constant int2 group
    key[0, 0, :, 1] = torch.linspace(-3e5, 3e5, T)           # int4, range > fp16 max * 15
    key[0, 0, :, 4] = torch.tensor([0.0, 0.5, 1.5, 2.5, 3.0] * 51 + [0.0])   # int2 ties
    key[0, 1, :, 0] = torch.randn(T) * 1e-30                 # tiny
    key[0, 1, :, 3] = torch.randn(T) * 1e5                   # fp16 tier overflows
    key[0, 1, :, 7] = -0.0
    key[0, 1, 5, 8] = 3e38                                    # range overflows float: a = inf
    key[0, 1, 6, 8] = -3e38
    key = key.bfloat16()
    value = (torch.randn(1, 2, T, D) * torch.logspace(-6, 6, D)).bfloat16()
    value[0, 0, 3] = 1.0
    value[0, 1, 9, :64] = 2e38
    value[0, 1, 9, 64:] = -2e38
    mgr = PackedKVManager([levels], 2, 2, D, 128, 128, 128, 2, gpu)
    mgr.commit(0, key.to(gpu), value.to(gpu))
    store = oracle_store(levels, f32(key[0]), f32(value[0]), 128, 128, 128, 2)
    assert_history_equal(mgr.layers[0], 0, store)


def test_division_sensitive_ties_on_device(gpu):
    """Groups where (x-lo)/s is exactly k+0.5 after IEEE division (x*(1/s) would round up)."""
    cases = [(1081804425, 1135190891), (1090252937, 1154556202), (1092564827, 1153771404)]
    D, T = 128, 128
    key = torch.zeros(1, 1, T, D, dtype=torch.float32)
    for i, (sb, db) in enumerate(cases):
        s = np.array([sb], np.uint32).view(np.float32)[0]
        d = np.array([db], np.uint32).view(np.float32)[0]
        key[0, 0, 1, i] = float(d)
        key[0, 0, 2, i] = float(np.float32(s * np.float32(255)))
    levels = np.full((1, D), 2, np.int64)
    levels[0, 100:] = 0
    mgr = PackedKVManager([levels], 1, 1, D, 128, 128, 128, 2, gpu)
    mgr.commit(0, key.to(gpu), key.to(gpu))
    store = oracle_store(levels, key[0].numpy(), key[0].numpy())
    assert_history_equal(mgr.layers[0], 0, store)


def test_token_by_token_commit_matches_bulk(gpu):
    d = synth.make_layer(1, 8, 2, 128, 300, 2.5, seed=9)
    k, v = d.key.to(gpu), d.value.to(gpu)
    bulk = make_manager(d.levels, 8, 2, 128, gpu)
    bulk.commit(0, k, v)
    step = make_manager(d.levels, 8, 2, 128, gpu)
    step.commit(0, k[:, :, :5], v[:, :, :5])
    for t in range(5, 300):
        step.commit(0, k[:, :, t:t + 1], v[:, :, t:t + 1])
    store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]))
    assert_history_equal(bulk.layers[0], 0, store)
    assert_history_equal(step.layers[0], 0, store)
    assert step.seq_len == 300 and step.layers[0].hist_len == 256 and step.layers[0].tail_len == 44


def test_batched_ragged_commits_and_growth(gpu):
    """Batch of 3 with ragged prefills (130, 7, 511 tokens), then 200 one-token commits;
    capacity starts at one page and grows; every sequence matches its own oracle store, and
    the page-major Key scale/min copy matches the reference arrays after the growth."""
    n_kv, D = 2, 128
    lens = [130, 7, 511]
    steps = 200
    data = [synth.make_layer(1, 4, n_kv, D, 720, 2.5, seed=20 + i) for i in range(3)]
    levels = data[0].levels
    mgr = PackedKVManager([levels], 4, n_kv, D, 128, 128, 128, 2, gpu, batch_size=3, capacity_tokens=128)
    layer = mgr.layers[0]
    pad = max(lens)
    k0 = torch.zeros(3, n_kv, pad, D, dtype=torch.bfloat16)
    v0 = torch.zeros_like(k0)
    for b in range(3):
        k0[b, :, :lens[b]] = data[b].key[0, :, :lens[b]]
        v0[b, :, :lens[b]] = data[b].value[0, :, :lens[b]]
    mgr.commit(0, k0.to(gpu), v0.to(gpu), lengths=lens)
    for t in range(steps):
        kt = torch.stack([data[b].key[0, :, lens[b] + t] for b in range(3)])[:, :, None].to(gpu)
        vt = torch.stack([data[b].value[0, :, lens[b] + t] for b in range(3)])[:, :, None].to(gpu)
        mgr.commit(0, kt, vt)
    for b in range(3):
        n = lens[b] + steps
        store = oracle_store(levels, f32(data[b].key[0, :, :n]), f32(data[b].value[0, :, :n]))
        assert_history_equal(layer, b, store)
        _check_page_copy(layer, b)  # the page-major scale/min copy survives every growth
    assert layer.capacity >= 640


def test_quantize_page_functions_match_oracle(gpu):
    d = synth.make_layer(1, 4, 4, 128, 128, 2.5, seed=3)
    table = pl.tier_tables(torch.as_tensor(d.levels).to(gpu))
    table2 = dict(table["tiers"])
    table2["tier"] = table["tier"]
    ours = pl.quantize_key_page(d.key[0].to(gpu), table2, 128)
    ref = ol.quantize_key_page(f32(d.key[0]), ol.layer_table(d.levels), 128)
    for t in range(3):
        for name in ("code", "scale", "min"):
            assert np.array_equal(ours[t][name].cpu().numpy().view(np.uint8), ref[t][name].view(np.uint8))
    assert np.array_equal(ours[3]["value"].cpu().numpy().view(np.uint16), ref[3]["value"].view(np.uint16))
    vo = pl.quantize_value_page(d.value[0].to(gpu), 2, 128)
    vr = ol.quantize_value_page(f32(d.value[0]), 2, 128)
    for name in ("code", "scale", "min"):
        assert np.array_equal(vo[name].cpu().numpy().view(np.uint8), vr[name].view(np.uint8))
    # dequantisers on the device vs the oracle: bit-exact float32
    kd = pl.dequantize_key(128, table2, ours, 128)
    assert np.array_equal(kd.cpu().numpy(), ol.dequantize_key(128, ol.layer_table(d.levels), ref, 128))
    vd = pl.dequantize_value(vo, 128, 128, 2, 128)
    assert np.array_equal(vd.cpu().numpy(), ol.dequantize_value(vr, 128, 128, 2, 128))


def test_cpu_tensors_raise(gpu):
    d = synth.make_layer(1, 4, 4, 128, 128, 2.5, seed=3)
    table = pl.tier_tables(torch.as_tensor(d.levels))
    t2 = dict(table["tiers"])
    t2["tier"] = table["tier"]
    with pytest.raises(RuntimeError, match="ROCm"):
        pl.quantize_key_page(d.key[0], t2, 128)
    with pytest.raises(RuntimeError, match="ROCm"):
        PackedKVManager([d.levels], 4, 4, 128, 128, 128, 128, 2, "cpu")


def _sm_blocks(words):
    """First block of each integer tier and the block count of a page's k_sm_page block."""
    steps = [2 * -(-words[0] // 4), -(-words[1] // 4), -(-(-(-words[2] // 2)) // 4)]
    return [0, 4 * steps[0], 4 * (steps[0] + steps[1])], 4 * sum(steps)


def _check_page_copy(layer, b):
    """Every page's k_sm_page block holds, per integer tier, exactly the reference arrays' fp16
    (scale, min) pairs of the head's real channels and (1.0, 0.0) at every other position of the
    tier's blocks (the positions themselves are what the decode parity tests pin: the matrix-core
    kernel reads the Key scales only from this copy)."""
    hk, _ = layer.export_reference(b)
    copy = layer.page_scale_copy(b).cpu().numpy().view(np.uint16)      # [n_kv, pages, 16 * nb]
    blk0, nb = _sm_blocks(layer.words)
    ends = blk0[1:] + [nb]
    counts = [layer.table[t]["count"].cpu().numpy() for t in range(3)]
    for h in range(layer.n_kv):
        for p in range(copy.shape[1]):
            blocks = copy[h, p].reshape(nb, 2, 8)                         # [block][scale, min][8]
            for t in range(3):
                seg = blocks[blk0[t]:ends[t]]
                got = sorted(zip(seg[:, 0].reshape(-1).tolist(), seg[:, 1].reshape(-1).tolist()))
                cnt = int(counts[t][h])
                sc = hk[t]["scale"][h, :cnt, p].cpu().numpy().view(np.uint16).tolist()
                mn = hk[t]["min"][h, :cnt, p].cpu().numpy().view(np.uint16).tolist()
                want = sorted(list(zip(sc, mn)) + [(0x3C00, 0)] * (seg.shape[0] * 8 - cnt))
                assert got == want, (h, p, t)


@pytest.mark.parametrize("path", ["fast", "generic", "deferred"])
def test_page_major_scale_copy_matches_reference_arrays(gpu, path):
    """The page-major Key scale/min copy written by the fast packer (bf16 pages), the generic
    packer (float32 pages) and the one-launch deferred flush (lf_pack_pages_multi) against the
    reference-layout arrays of the same pages, for ragged heads (c2's tier sampler)."""
    n_kv, D, B = 4, 128, 2
    lv = synth.sample_tier_levels(n_kv, D, 2.5, seed=77)
    d = synth.make_layer(B, 28, n_kv, D, 3 * 128 + 50, 2.5, seed=77)
    d.levels = lv
    key = d.key.float() if path == "generic" else d.key
    value = d.value.float() if path == "generic" else d.value
    m = PackedKVManager([lv, lv], 28, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B,
                        defer_flush=path == "deferred")
    if path == "deferred":
        # a decode loop: every layer commits the token, then one flush packs the step's pages of
        # both layers in one lf_pack_pages_multi launch
        kg, vg = key.to(gpu), value.to(gpu)
        for t in range(3 * 128 + 50):
            for layer in range(2):
                m.commit(layer, kg[:, :, t:t + 1], vg[:, :, t:t + 1])
            m.flush_pending()
    else:
        for layer in range(2):
            m.commit(layer, key.to(gpu), value.to(gpu))
    torch.cuda.synchronize()
    for layer in range(2):
        for b in range(B):
            assert m.layers[layer].hist_lens[b] == 3 * 128
            _check_page_copy(m.layers[layer], b)
