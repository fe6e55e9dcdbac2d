"""Device layout helpers and the shapes that need padded Value rows, against the oracle.

* ``asymmetric_codes`` / ``pack_ints`` / ``unpack_ints`` (reference
  src/logitfill/packed/layout.py:12-46) bit-exact against the oracle's restatement, which the
  golden vectors of the reference packer pin;
* the reference's own pack/dequantise test shape (tests/test_logitfill_offline.py:127-145:
  two heads, a 16-token page, head_dim 8, Key and Value groups of 8, all-int2 Keys), whose
  Value rows of 16 bits are padded to one word (layout.py:27-29);
* decode at head_dim 8 .. 512 and with 16 Value groups per token (v_group 8 at head_dim 128),
  served by the general HIP kernel, against the oracle's dense path.
"""
import numpy as np
import pytest
import torch

from logitfill_amd import synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed import layout as dl
from logitfill_amd.packed import reference as dref
from oracle import layout as ol
from tests.helpers import assert_decode_close, assert_history_equal, f32, oracle_decode, oracle_store

pytestmark = pytest.mark.gpu


def _groups(rng, n, group, dtype):
    x = rng.standard_normal((n, group)).astype(np.float32) * rng.lognormal(0, 1, (n, 1)).astype(np.float32)
    x[0] = 0.75                                    # constant group: scale clamps to 1e-5
    x[1, :] = np.linspace(-1.5, 1.5, group)        # a ramp with exact ties
    x[2] *= 1e-7                                   # range below the 1e-5 scale floor
    t = torch.from_numpy(x).to(dtype)
    return t, t.float().numpy()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("group,bits", [(8, 2), (128, 2), (7, 4), (64, 8), (33, 3)])
def test_asymmetric_codes_bit_exact(gpu, dtype, group, bits):
    rng = np.random.default_rng(group * 10 + bits)
    t, x = _groups(rng, 257, group, dtype)
    codes, scale, low = dl.asymmetric_codes(t.to(gpu), bits)
    want_c, want_s, want_l = ol.asymmetric_codes(x, bits)
    assert codes.dtype == torch.int32 and tuple(codes.shape) == x.shape
    assert np.array_equal(codes.cpu().numpy(), want_c)
    assert np.array_equal(scale.cpu().numpy().view(np.uint32), want_s.view(np.uint32))
    assert np.array_equal(low.cpu().numpy().view(np.uint32), want_l.view(np.uint32))


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8, 10, 16, 20, 32])
@pytest.mark.parametrize("n", [1, 5, 16, 17, 40, 128])
def test_pack_and_unpack_ints_bit_exact(gpu, bits, n):
    """Every width of the reference's pack_ints (layout.py:21-46): per = 32 // bits slots a word,
    so widths that do not divide 32 leave the top bits of each word zero (3 bits: ten slots,
    bits 30-31 unused) and widths above 16 take one slot a word (bits 32: the words themselves)."""
    rng = np.random.default_rng(bits * 1000 + n)
    codes = rng.integers(0, min(1 << bits, 1 << 31), size=(3, 5, n), dtype=np.int64).astype(np.int32)
    words = dl.pack_ints(torch.from_numpy(codes).to(gpu), bits)
    want = ol.pack_ints(codes, bits)
    assert tuple(words.shape) == want.shape
    assert np.array_equal(words.cpu().numpy(), want)
    back = dl.unpack_ints(words, n, bits)
    assert np.array_equal(back.cpu().numpy(), codes)
    # the top slot of a full word may set the sign bit; unpacking still returns the code
    assert np.array_equal(dl.unpack_ints(words, min(n, 3), bits).cpu().numpy(), codes[..., :min(n, 3)])


def test_reference_offline_test_shape_pack_and_dequantise(gpu):
    """Reference tests/test_logitfill_offline.py:127-145 on the device: a [2, 16, 8] float32 page,
    all-int2 Key levels, Key groups of 8 tokens, int2 Values in groups of 8 channels (16-bit
    rows, one padded word).  Codes, scales and mins are bit-exact against the oracle; the
    dequantised tensors equal the oracle's."""
    torch.manual_seed(0)
    page = torch.randn(2, 16, 8)
    levels = torch.zeros(2, 8, dtype=torch.int64)
    built = dl.tier_tables(levels)
    table = dict(built["tiers"])
    table["tier"] = built["tier"]
    packed = dl.quantize_key_page(page.to(gpu), table, group_size=8)
    otable = ol.layer_table(levels.numpy())
    want = ol.quantize_key_page(page.numpy(), otable, 8)
    for name in ("code", "scale", "min"):
        assert np.array_equal(packed[0][name].cpu().numpy().view(np.uint8), want[0][name].view(np.uint8)), name
    restored = dl.dequantize_key(16, table, packed, group_size=8)
    assert np.array_equal(restored.cpu().numpy(), ol.dequantize_key(16, otable, want, 8))

    values = dl.quantize_value_page(page.to(gpu), bits=2, group_size=8)
    want_v = ol.quantize_value_page(page.numpy(), 2, 8)
    assert tuple(values["code"].shape) == (2, 16, 1) == want_v["code"].shape
    for name in ("code", "scale", "min"):
        assert np.array_equal(values[name].cpu().numpy().view(np.uint8), want_v[name].view(np.uint8)), name
    restored_v = dl.dequantize_value(values, 16, 8, bits=2, group_size=8)
    assert np.array_equal(restored_v.cpu().numpy(), ol.dequantize_value(want_v, 16, 8, 2, 8))


@pytest.mark.parametrize("D,page,kg,vg,bit_v", [(8, 16, 8, 8, 2), (20, 16, 16, 10, 4), (6, 32, 32, 3, 8),
                                                 (12, 32, 16, 4, 8)])
def test_padded_value_rows_through_the_cache(gpu, D, page, kg, vg, bit_v):
    """Commit loops through PackedKVManager with Value rows of 16, 80 and 48 bits (padded to 1, 3
    and 2 words) and one of 96 bits (3 whole words): the device history equals the oracle store
    bit for bit."""
    n_kv = 2
    rng = np.random.default_rng(D)
    levels = rng.integers(0, 4, size=(n_kv, D))
    key = torch.randn(1, n_kv, 5 * page + 3, D, generator=torch.Generator().manual_seed(D)).to(torch.bfloat16)
    value = torch.randn(1, n_kv, 5 * page + 3, D, generator=torch.Generator().manual_seed(D + 1)).to(torch.bfloat16)
    mgr = PackedKVManager([levels], 2 * n_kv, n_kv, D, page, kg, vg, bit_v, gpu)
    for t0, t1 in ((0, 7), (7, page + 2), (page + 2, 5 * page + 3)):
        mgr.commit(0, key[:, :, t0:t1].to(gpu), value[:, :, t0:t1].to(gpu))
    store = oracle_store(levels, f32(key[0]), f32(value[0]), page, kg, vg, bit_v)
    assert_history_equal(mgr.layers[0], 0, store)


@pytest.mark.parametrize("D,n_q,n_kv,page,vg", [(8, 2, 1, 16, 8), (16, 6, 2, 32, 16), (32, 4, 1, 64, 8),
                                               (512, 8, 2, 128, 128), (128, 14, 2, 128, 8)])
def test_decode_general_shapes_against_oracle(gpu, D, n_q, n_kv, page, vg):
    """The general kernel at head_dim 8, 16, 32 and 512 and with 16 Value groups per token
    (v_group 8 at head_dim 128): the decode of a ragged commit sequence (pages + residual +
    the new token) meets the north-star bar against the oracle.  No call takes the dense path."""
    dref.DENSE_FALLBACKS.clear()
    rng = np.random.default_rng(D + vg)
    levels = rng.choice(4, size=(n_kv, D), p=[0.6, 0.25, 0.1, 0.05])
    T = 3 * page + page // 2 + 1
    g = torch.Generator().manual_seed(D * 7 + vg)
    key = torch.randn(1, n_kv, T, D, generator=g).to(torch.bfloat16)
    value = torch.randn(1, n_kv, T, D, generator=g).to(torch.bfloat16)
    q = (torch.randn(1, n_q, 1, D, generator=g) * D ** -0.5).to(torch.bfloat16)
    kn = torch.randn(1, n_kv, 1, D, generator=g).to(torch.bfloat16)
    vn = torch.randn(1, n_kv, 1, D, generator=g).to(torch.bfloat16)
    mgr = PackedKVManager([levels], n_q, n_kv, D, page, page, vg, 2, gpu)
    mgr.commit(0, key.to(gpu), value.to(gpu))
    out = dref.packed_attention(mgr, 0, q.to(gpu), kn.to(gpu), vn.to(gpu), D ** -0.5)
    torch.cuda.synchronize()
    assert not dref.DENSE_FALLBACKS, dict(dref.DENSE_FALLBACKS)
    store = oracle_store(levels, f32(key[0]), f32(value[0]), page, page, vg, 2)
    ref = oracle_decode(store, f32(q[0, :, 0]), f32(kn[0, :, 0]), f32(vn[0, :, 0]), D ** -0.5, n_q, n_kv)
    assert_decode_close(out[0, :, 0], ref)


def test_unsupported_shapes_take_the_counted_dense_path(gpu):
    """Values at 4 and 8 bits are outside the decode kernels (the reference kernel also takes
    int2 Values only, reference.py:62): packed_attention runs the dense dequantise-then-attend
    path on the device, counts the call, and matches the oracle; with LOGITFILL_AMD_STRICT=1 it
    raises instead.  (Any GQA group stays on the kernels: tests/test_gpu_rows.py.)"""
    import os

    dref.DENSE_FALLBACKS.clear()
    D, n_kv = 64, 1
    for n_q, bit_v in ((2, 4), (24, 8)):
        levels = np.zeros((n_kv, D), dtype=np.int64)
        T = 2 * 64 + 5
        g = torch.Generator().manual_seed(n_q)
        key = torch.randn(1, n_kv, T, D, generator=g).to(torch.bfloat16)
        value = torch.randn(1, n_kv, T, D, generator=g).to(torch.bfloat16)
        q = (torch.randn(1, n_q, 1, D, generator=g) * D ** -0.5).to(torch.bfloat16)
        kn = torch.randn(1, n_kv, 1, D, generator=g).to(torch.bfloat16)
        vn = torch.randn(1, n_kv, 1, D, generator=g).to(torch.bfloat16)
        mgr = PackedKVManager([levels], n_q, n_kv, D, 64, 64, 64, bit_v, gpu)
        mgr.commit(0, key.to(gpu), value.to(gpu))
        with pytest.warns(RuntimeWarning):
            dref._WARNED.clear()
            out = dref.packed_attention(mgr, 0, q.to(gpu), kn.to(gpu), vn.to(gpu), D ** -0.5)
        store = oracle_store(levels, f32(key[0]), f32(value[0]), 64, 64, 64, bit_v)
        ref = oracle_decode(store, f32(q[0, :, 0]), f32(kn[0, :, 0]), f32(vn[0, :, 0]), D ** -0.5, n_q, n_kv)
        assert_decode_close(out[0, :, 0], ref)
        os.environ["LOGITFILL_AMD_STRICT"] = "1"
        try:
            with pytest.raises(RuntimeError):
                dref.packed_attention(mgr, 0, q.to(gpu), kn.to(gpu), vn.to(gpu), D ** -0.5)
        finally:
            del os.environ["LOGITFILL_AMD_STRICT"]
    assert sum(dref.DENSE_FALLBACKS.values()) == 2
