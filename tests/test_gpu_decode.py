"""GPU parity of the decode-attention path against the oracle's dense
dequantise-then-attend path (reference src/logitfill/packed/reference.py:30-56):
bf16 output within max-abs 2e-3 and rel-L2 1e-3 (fp32 accumulation), on the
same seeded inputs; plus split-count invariance and the reference's own
kernel-test shape."""
import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import decode_into, packed_attention, reference_attention
from oracle import attention as oatt
from tests.helpers import assert_decode_close, f32, oracle_decode, oracle_store

pytestmark = pytest.mark.gpu

KERNELS = {"valu": _native.KERNEL_VALU, "mfma": _native.KERNEL_MFMA, "auto": _native.KERNEL_AUTO}


def build(d, pages, tails, n_q, n_kv, D, dev, page=128, kg=128, vg=128):
    """Manager whose sequence b holds pages[b] packed pages then tails[b] residual tokens of d."""
    B = len(pages)
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, page, kg, vg, 2, dev, batch_size=B)
    lens = [p * page + t for p, t in zip(pages, tails)]
    mgr.commit(0, d.key[:, :, :max(lens)].to(dev), d.value[:, :, :max(lens)].to(dev), lengths=lens)
    return mgr, lens


def oracle_out(d, b, n, n_q, n_kv, scaling, page=128, kg=128, vg=128):
    store = oracle_store(d.levels, f32(d.key[b, :, :n]), f32(d.value[b, :, :n]), page, kg, vg, 2)
    return oracle_decode(store, f32(d.query[b]), f32(d.key_new[b]), f32(d.value_new[b]), scaling, n_q, n_kv)


def run(mgr, d, dev, scaling, kernel, pages_per_split=None, out_dtype=None):
    q = d.query.to(dev)
    out = torch.empty(q.shape, dtype=out_dtype or q.dtype, device=dev)
    decode_into(mgr, 0, q, d.key_new.to(dev), d.value_new.to(dev), scaling, out, kernel=kernel,
                pages_per_split=pages_per_split)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kernel", list(KERNELS))
def test_config0_decode(gpu, kernel):
    """1 seq, 4 kv / 28 q heads, 8 pages + the new token, target 2.5."""
    d = synth.make_layer(1, 28, 4, 128, 1024, 2.5, seed=0)
    mgr, lens = build(d, [8], [0], 28, 4, 128, gpu)
    out = run(mgr, d, gpu, 128 ** -0.5, KERNELS[kernel])
    assert_decode_close(out[0], oracle_out(d, 0, 1024, 28, 4, 128 ** -0.5))


@pytest.mark.parametrize("kernel", list(KERNELS))
def test_ragged_batch_decode(gpu, kernel):
    """Ragged batch (GQA 5): histories of 0..12 pages, residual pages of 0..127 tokens."""
    pages, tails = [0, 1, 5, 12, 3], [3, 0, 127, 50, 1]
    d = synth.make_layer(5, 10, 2, 128, 12 * 128 + 127, 2.5, seed=4)
    mgr, lens = build(d, pages, tails, 10, 2, 128, gpu)
    out = run(mgr, d, gpu, 0.0883, KERNELS[kernel])
    for b in range(5):
        assert_decode_close(out[b], oracle_out(d, b, lens[b], 10, 2, 0.0883))


@pytest.mark.parametrize("kernel", list(KERNELS))
def test_split_count_invariance(gpu, kernel):
    d = synth.make_layer(2, 14, 2, 128, 20 * 128 + 9, 3.0, seed=8)
    mgr, lens = build(d, [20, 13], [9, 77], 14, 2, 128, gpu)
    outs = [run(mgr, d, gpu, 0.09, KERNELS[kernel], pages_per_split=s, out_dtype=torch.float32)
            for s in (1, 3, 64)]
    # the VALU path is fp32 throughout; the MFMA path rounds hi/lo fp16 operands (~22 bits) and
    # accumulates Value codes as 4 + c (the offset cancels against the per-token constant), so
    # its result moves by a few 1e-5 relative with the split pattern (a merge error is >> 1e-3)
    rel_bar = 2e-6 if kernel == "valu" else 1e-4
    for o in outs[1:]:
        rel = float((o - outs[0]).norm() / outs[0].norm())
        assert rel <= rel_bar, f"split-count change moved the output by {rel:.3g} (bar {rel_bar})"
    for b in range(2):
        ref = oracle_out(d, b, lens[b], 14, 2, 0.09)
        assert_decode_close(outs[0][b], ref, out_dtype="fp32")


def test_reference_kernel_test_shape(gpu):
    """tests/test_logitfill_offline.py:187-219: D 64, n_q = n_kv = 1, page = groups = 64,
    all four tiers, float32 data; the reference compares kernel vs dense at 1e-3."""
    g = torch.Generator().manual_seed(0)
    levels = torch.randint(0, 4, (1, 64), generator=g)
    key = torch.randn(1, 1, 64, 64, generator=g)
    value = torch.randn(1, 1, 64, 64, generator=g)
    mgr = PackedKVManager([levels], 1, 1, 64, 64, 64, 64, 2, gpu)
    mgr.commit(0, key.to(gpu), value.to(gpu))
    query = torch.randn(1, 1, 1, 64, generator=g)
    new_k = torch.randn(1, 1, 1, 64, generator=g)
    new_v = torch.randn(1, 1, 1, 64, generator=g)
    fast = packed_attention(mgr, 0, query.to(gpu), new_k.to(gpu), new_v.to(gpu), scaling=64 ** -0.5)
    slow = reference_attention(mgr, 0, query.to(gpu), new_k.to(gpu), new_v.to(gpu), scaling=64 ** -0.5)
    assert fast.shape == (1, 1, 1, 64) and fast.dtype == torch.float32
    assert torch.allclose(fast.float(), slow.float(), atol=1e-3, rtol=1e-3)
    store = oracle_store(levels.numpy(), key[0].numpy(), value[0].numpy(), 64, 64, 64, 2)
    ref = oatt.reference_attention(store, query[0].numpy(), new_k[0].numpy(), new_v[0].numpy(), 64 ** -0.5, 1, 1)
    assert_decode_close(fast[0, :, 0], ref[:, 0], out_dtype="fp32", max_abs=1e-5, rel_l2=1e-5)


def test_query_not_8_byte_aligned(gpu):
    """A bf16 query whose rows start 2 bytes past an 8-byte boundary (a view into a larger
    buffer): the kernel's 8-byte q loads give way to element loads, same result."""
    d = synth.make_layer(1, 8, 2, 128, 3 * 128 + 5, 2.5, seed=13)
    mgr, lens = build(d, [3], [5], 8, 2, 128, gpu)
    q = d.query.to(gpu)
    buf = torch.empty(q.numel() + 1, dtype=q.dtype, device=gpu)
    qv = buf[1:].view(q.shape)
    qv.copy_(q)
    assert qv.data_ptr() % 8 == 2
    outs = []
    for qq in (q, qv):
        out = torch.empty(q.shape, dtype=torch.float32, device=gpu)
        decode_into(mgr, 0, qq, d.key_new.to(gpu), d.value_new.to(gpu), 0.1, out)
        outs.append(out)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.float32])
def test_query_and_output_dtypes(gpu, q_dtype):
    d = synth.make_layer(1, 8, 2, 128, 3 * 128 + 5, 2.5, seed=12)
    mgr, lens = build(d, [3], [5], 8, 2, 128, gpu)
    q = d.query.to(q_dtype).to(gpu)
    out = torch.empty(q.shape, dtype=q_dtype, device=gpu)
    decode_into(mgr, 0, q, d.key_new.to(gpu), d.value_new.to(gpu), 0.1, out)
    torch.cuda.synchronize()
    ref = oracle_decode(oracle_store(d.levels, f32(d.key[0, :, :lens[0]]), f32(d.value[0, :, :lens[0]])),
                        f32(q[0]), f32(d.key_new[0]), f32(d.value_new[0]), 0.1, 8, 2)
    assert_decode_close(out[0], ref, out_dtype="fp16" if q_dtype == torch.float16 else "fp32")


def test_decode_commit_loop_crossing_flushes(gpu):
    """Model order (attention, then commit; reference models/qwen2_attention.py:244-253)
    for 140 decode steps starting 3 tokens before a page boundary."""
    n_q, n_kv, D = 6, 2, 128
    total = 128 + 125 + 140 + 1
    d = synth.make_layer(1, n_q, n_kv, D, total, 2.5, seed=31)
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu)
    k, v = d.key.to(gpu), d.value.to(gpu)
    mgr.commit(0, k[:, :, :253], v[:, :, :253])
    # unscaled N(0,1) queries: peaked attention, outputs of order 1 (bf16 ulp > 2e-3)
    qs = torch.randn(140, 1, n_q, 1, D, generator=torch.Generator().manual_seed(1)).bfloat16()
    for step in range(140):
        pos = 253 + step
        out = packed_attention(mgr, 0, qs[step].to(gpu), k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], D ** -0.5)
        if step in (0, 2, 3, 139):
            out32 = torch.empty(1, n_q, D, dtype=torch.float32, device=gpu)
            decode_into(mgr, 0, qs[step][:, :, 0].contiguous().to(gpu), k[:, :, pos].contiguous(),
                        v[:, :, pos].contiguous(), D ** -0.5, out32)
            store = oracle_store(d.levels, f32(d.key[0, :, :pos]), f32(d.value[0, :, :pos]))
            ref = oatt.reference_attention(store, f32(qs[step][0]), f32(d.key[0, :, pos:pos + 1]),
                                           f32(d.value[0, :, pos:pos + 1]), D ** -0.5, n_q, n_kv)
            assert_decode_close(out[0, :, 0], ref[:, 0])
            assert_decode_close(out32[0], ref[:, 0], out_dtype="fp32")
        mgr.commit(0, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1])
    assert mgr.layers[0].hist_len == 384 and mgr.layers[0].tail_len == 9


def test_multi_token_query_small_group(gpu):
    """q_len > 1 (chunked scoring) with the right-aligned causal mask (rows 2 * 3 <= 16: kernel)."""
    n_q, n_kv, D = 4, 2, 128
    d = synth.make_layer(1, n_q, n_kv, D, 2 * 128 + 30, 2.5, seed=40)
    mgr, lens = build(d, [2], [20], n_q, n_kv, D, gpu)
    q = torch.randn(1, n_q, 3, D, generator=torch.Generator().manual_seed(2)).bfloat16()
    kn, vn = d.key[:, :, 276:279], d.value[:, :, 276:279]
    out = packed_attention(mgr, 0, q.to(gpu), kn.to(gpu), vn.to(gpu), 0.1)
    store = oracle_store(d.levels, f32(d.key[0, :, :276]), f32(d.value[0, :, :276]))
    ref = oatt.reference_attention(store, f32(q[0]), f32(kn[0]), f32(vn[0]), 0.1, n_q, n_kv)
    assert_decode_close(out[0], ref)


def test_device_dequantize_matches_oracle(gpu):
    d = synth.make_layer(2, 8, 4, 128, 5 * 128, 2.5, seed=50)
    mgr, lens = build(d, [5, 2], [0, 11], 8, 4, 128, gpu)
    for b in range(2):
        kd, vd = mgr.layers[0].dequantize(b)
        store = oracle_store(d.levels, f32(d.key[b, :, :lens[b]]), f32(d.value[b, :, :lens[b]]))
        ok, ov = store.dequantize()
        assert np.array_equal(kd.cpu().numpy(), ok) and np.array_equal(vd.cpu().numpy(), ov)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("g,levels_kind", [(1, "uniform"), (8, "uniform"), (7, "fp16heavy"), (5, "int8heavy")])
def test_tier_mix_and_group_sizes(gpu, kernel, g, levels_kind):
    """Tier tables far from the sampler's (wide int8 / fp16 tiers, every K-step path) and
    GQA groups 1..8; 37-page histories split 40 pages per item (> one 16-page scale chunk)."""
    n_kv, D = 2, 128
    rng = np.random.default_rng(g)
    if levels_kind == "uniform":
        levels = rng.integers(0, 4, (n_kv, D))
    elif levels_kind == "fp16heavy":
        levels = rng.choice(4, (n_kv, D), p=[0.2, 0.1, 0.1, 0.6])
    else:
        levels = rng.choice(4, (n_kv, D), p=[0.1, 0.2, 0.6, 0.1])
    d = synth.make_layer(2, g * n_kv, n_kv, D, 37 * 128 + 127, 2.5, seed=60 + g)
    d.levels = levels
    mgr, lens = build(d, [37, 20], [127, 0], g * n_kv, n_kv, D, gpu)
    out = run(mgr, d, gpu, D ** -0.5, KERNELS[kernel], pages_per_split=40)
    for b in range(2):
        assert_decode_close(out[b], oracle_out(d, b, lens[b], g * n_kv, n_kv, D ** -0.5))


def test_mfma_kernel_rejects_unsupported_shape(gpu):
    """The MFMA kernel serves D 128 / page 128; an explicit request elsewhere is an error."""
    g = torch.Generator().manual_seed(0)
    levels = torch.randint(0, 4, (1, 64), generator=g)
    mgr = PackedKVManager([levels], 1, 1, 64, 64, 64, 64, 2, gpu)
    mgr.commit(0, torch.randn(1, 1, 64, 64, generator=g).to(gpu), torch.randn(1, 1, 64, 64, generator=g).to(gpu))
    q = torch.randn(1, 1, 64, device=gpu)
    out = torch.empty_like(q)
    with pytest.raises(_native.LFError):
        decode_into(mgr, 0, q, q.clone(), q.clone(), 0.125, out, kernel=_native.KERNEL_MFMA)


@pytest.mark.parametrize("kernel", ["valu", "mfma"])
@pytest.mark.parametrize("profile", ["ramp", "spike"])
def test_score_growth_across_pages(gpu, kernel, profile):
    """Keys scaled per token so the page maxima climb by far more than the kernels' lazy
    rescale headroom (2^8) from page to page ("ramp"), or jump once mid-sequence and fall back
    ("spike"): the running reference moves on later pages of one split item, so O, l and the
    midpoint sums are rescaled inside the page loop, not only at the first page."""
    n_q, n_kv, D, pages = 8, 2, 128, 24
    T = pages * 128 + 40
    d = synth.make_layer(2, n_q, n_kv, D, T, 2.5, seed=70)
    t = torch.arange(T, dtype=torch.float32)
    if profile == "ramp":
        gain = 0.05 + 6.0 * t / T
    else:
        gain = torch.full((T,), 0.3)
        gain[9 * 128:10 * 128] = 6.0
    d.key = (d.key.float() * gain[None, None, :, None]).bfloat16()
    d.query = (d.query.float() * 4.0).bfloat16()
    mgr, lens = build(d, [pages, pages - 5], [40, 3], n_q, n_kv, D, gpu)
    for pps in (64, 5):
        out = run(mgr, d, gpu, D ** -0.5, KERNELS[kernel], pages_per_split=pps)
        for b in range(2):
            assert_decode_close(out[b], oracle_out(d, b, lens[b], n_q, n_kv, D ** -0.5))


@pytest.mark.parametrize("g,q_len,tails", [(2, 2, [0, 63]), (4, 3, [127, 5]), (2, 8, [61, 0]), (7, 3, [9, 100])])
def test_multi_token_packed_decode(gpu, g, q_len, tails):
    """q_len new tokens per sequence (speculative decoding / chunked scoring, reference
    reference.py:18-27,48): query token j sees the history, the tail and new tokens 0..j.
    ``packed_attention`` keeps every case on the decode kernels (no dense fallback), and both
    kernels meet the bar with split items (the residual riding with each sequence's first
    item); rows beyond a workgroup's tile (the matrix-core kernel's 8, the VALU kernel's 16)
    run as further row tiles."""
    from logitfill_amd.packed.reference import DENSE_FALLBACKS

    n_kv, D = 2, 128
    n_q = g * n_kv
    pages = [6, 3]
    T = max(p * 128 + t for p, t in zip(pages, tails)) + q_len
    d = synth.make_layer(2, n_q, n_kv, D, T, 2.5, seed=100 + q_len)
    mgr, lens = build(d, pages, tails, n_q, n_kv, D, gpu)
    q = torch.randn(2, n_q, q_len, D, generator=torch.Generator().manual_seed(q_len)).bfloat16()
    kn = torch.stack([d.key[b, :, lens[b]:lens[b] + q_len] for b in range(2)])
    vn = torch.stack([d.value[b, :, lens[b]:lens[b] + q_len] for b in range(2)])
    before = dict(DENSE_FALLBACKS)
    out = packed_attention(mgr, 0, q.to(gpu), kn.to(gpu), vn.to(gpu), D ** -0.5)
    torch.cuda.synchronize()
    assert dict(DENSE_FALLBACKS) == before
    refs = []
    for b in range(2):
        store = oracle_store(d.levels, f32(d.key[b, :, :lens[b]]), f32(d.value[b, :, :lens[b]]))
        refs.append(oatt.reference_attention(store, f32(q[b]), f32(kn[b]), f32(vn[b]), D ** -0.5, n_q, n_kv))
        for j in range(q_len):
            assert_decode_close(out[b, :, j], refs[b][:, j])
    for kernel in (_native.KERNEL_MFMA, _native.KERNEL_VALU):
        out2 = torch.empty(2, n_q, q_len, D, dtype=torch.float32, device=gpu)
        decode_into(mgr, 0, q.to(gpu).contiguous(), kn.to(gpu).contiguous(), vn.to(gpu).contiguous(),
                    D ** -0.5, out2, kernel=kernel, pages_per_split=2)
        torch.cuda.synchronize()
        for b in range(2):
            for j in range(q_len):
                assert_decode_close(out2[b, :, j], refs[b][:, j], out_dtype="fp32")
