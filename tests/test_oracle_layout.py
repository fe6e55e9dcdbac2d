"""Pin the numpy oracle's packer and dequantiser (reference src/logitfill/packed/layout.py).

Known answers computed by hand, brute force with float64 arithmetic, and the
invariants the format guarantees; each is chosen so that a plausible mistake
(round-half-up, reciprocal division, transposed axes, wrong bit order, wrong
padding) fails at least one test.
"""
import numpy as np
import pytest

from oracle import layout

F32 = np.float32


def f16bits(x):
    return np.asarray(x, dtype=np.float16).view(np.uint16)


# ---- asymmetric_codes (layout.py:12-18) ----------------------------------------

def test_ramp_known_answer():
    codes, s, lo = layout.asymmetric_codes(np.array([[0, 1, 2, 3]], F32), 2)
    assert codes.tolist() == [[0, 1, 2, 3]]
    assert s.tolist() == [1.0] and lo.tolist() == [0.0]
    assert codes.dtype == np.int32 and s.dtype == np.float32


def test_ties_round_half_to_even():
    # (x - lo)/s = 0, .5, 1.5, 2.5, 3  ->  0, 0, 2, 2, 3 (half up would give 0,1,2,3,3)
    codes, s, lo = layout.asymmetric_codes(np.array([[0, 0.5, 1.5, 2.5, 3]], F32), 2)
    assert s.tolist() == [1.0]
    assert codes.tolist() == [[0, 0, 2, 2, 3]]


def test_constant_group_clamps_scale_to_1e5_floor():
    codes, s, lo = layout.asymmetric_codes(np.full((1, 8), 5.0, F32), 4)
    assert codes.tolist() == [[0] * 8]
    assert s[0] == F32(1e-5) and lo[0] == 5.0


def test_huge_range_clamps_scale_and_fp16_overflows():
    codes, s, lo = layout.asymmetric_codes(np.array([[0.0, 1e6]], F32), 2)
    assert s[0] == F32(1e5)                      # 1e6/3 clamped
    assert codes.tolist() == [[0, 3]]            # 1e6/1e5 = 10 clamped to qmax
    with np.errstate(over="ignore"):
        assert f16bits(s.astype(np.float16))[0] == 0x7C00   # fp16(1e5) = +inf


def test_scale_is_fp32_true_division_and_fp16_rne():
    codes, s, lo = layout.asymmetric_codes(np.array([[0, 1]], F32), 2)
    assert s[0] == F32(1) / F32(3)
    assert f16bits(s.astype(np.float16))[0] == 0x3555  # 0.33325, nearest fp16 to 1/3


def test_codes_match_correctly_rounded_division_bruteforce():
    """fl32(d/s) computed exactly in float64 (53 >= 2*24+2, so no double-rounding error)."""
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((4096, 16)) * rng.lognormal(0, 2, (4096, 1))).astype(F32)
    for bits in (2, 4, 8):
        qmax = (1 << bits) - 1
        codes, s, lo = layout.asymmetric_codes(x, bits)
        hi = x.max(-1)
        lo64 = x.min(-1)
        s_ref = np.clip((np.float64(hi - lo64) / qmax).astype(F32), F32(1e-5), F32(1e5))
        assert np.array_equal(s, s_ref)
        d = (x - lo64[:, None])                                   # float32 subtraction, as the reference
        q_exact = (d.astype(np.float64) / s_ref[:, None].astype(np.float64)).astype(F32)
        ref = np.clip(np.rint(q_exact), 0, qmax).astype(np.int32)
        assert np.array_equal(codes, ref)


def test_division_sensitive_known_answer():
    """(x - lo)/s lands exactly on k + 0.5: IEEE division gives the even code, while
    x * (1/s) rounds just above the tie and would give the odd one."""
    cases = [(1081804425, 1135190891, 86), (1090252937, 1154556202, 212), (1092564827, 1153771404, 158)]
    for sbits, dbits, even in cases:
        s = np.array([sbits], np.uint32).view(F32)[0]
        d = np.array([dbits], np.uint32).view(F32)[0]
        hi = F32(s * F32(255))
        codes, sc, lo = layout.asymmetric_codes(np.array([[0.0, d, hi]], F32), 8)
        assert sc[0] == s and lo[0] == 0.0
        assert codes[0, 1] == even
        assert np.rint(d * (F32(1) / s)) == even + 1


def test_code_range_invariant():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((100, 128)).astype(F32)
    for bits in (2, 4, 8):
        codes, _, _ = layout.asymmetric_codes(x, bits)
        assert codes.min() == 0 and codes.max() == (1 << bits) - 1


# ---- pack_ints / unpack_ints (layout.py:21-46) ---------------------------------

def test_pack_bit_positions_lsb_first():
    assert layout.pack_ints(np.array([[1, 2, 3]]), 2).tolist() == [[1 | 2 << 2 | 3 << 4]]
    top = np.zeros(16, np.int32)
    top[15] = 3
    assert layout.pack_ints(top[None], 2).view(np.uint32).tolist() == [[0xC0000000]]
    assert layout.pack_ints(np.array([[0, 0, 0, 0, 0, 0, 0, 9]]), 4).view(np.uint32).tolist() == [[9 << 28]]
    assert layout.pack_ints(np.array([[0x12, 0x34, 0x56, 0x78]]), 8).view(np.uint32).tolist() == [[0x78563412]]


def test_pack_pads_to_whole_words():
    codes = np.arange(17) % 4
    words = layout.pack_ints(codes[None], 2)
    assert words.shape == (1, 2)
    assert words[0, 1] == codes[16]
    assert layout.pack_ints(np.zeros((3, 0), np.int32), 2).shape == (3, 0)


def test_pack_unpack_roundtrip():
    rng = np.random.default_rng(3)
    for bits in (2, 4, 8):
        codes = rng.integers(0, 1 << bits, size=(5, 7, 37)).astype(np.int32)
        packed = layout.pack_ints(codes, bits)
        assert packed.dtype == np.int32 and packed.shape[-1] == -(-37 // (32 // bits))
        assert np.array_equal(layout.unpack_ints(packed, 37, bits), codes)


# ---- tier_tables (layout.py:49-68) ----------------------------------------------

LEVELS = np.array([[0, 3, 1, 0], [2, 0, 0, 1]])


def test_tier_tables_known_answer():
    t = layout.tier_tables(LEVELS)
    tiers = t["tiers"]
    assert tiers[0]["width"] == 2 and tiers[0]["index"].tolist() == [[0, 3], [1, 2]]
    assert tiers[0]["count"].tolist() == [2, 2]
    assert tiers[0]["local"].tolist() == [[0, -1, -1, 1], [-1, 0, 1, -1]]
    assert tiers[1]["index"].tolist() == [[2], [3]] and tiers[1]["count"].tolist() == [1, 1]
    assert tiers[2]["width"] == 1 and tiers[2]["index"].tolist() == [[0], [0]]
    assert tiers[2]["count"].tolist() == [0, 1]
    assert tiers[3]["index"].tolist() == [[1], [0]] and tiers[3]["count"].tolist() == [1, 0]
    assert t["tier"].dtype == np.int32 and t["tier"].tolist() == LEVELS.tolist()


def test_tier_tables_invariants_random():
    rng = np.random.default_rng(4)
    lv = rng.integers(0, 4, size=(6, 128))
    t = layout.tier_tables(lv)["tiers"]
    for code in range(4):
        for h in range(6):
            n = int(t[code]["count"][h])
            chans = t[code]["index"][h, :n]
            assert np.all(np.diff(chans) > 0)
            assert np.all(lv[h, chans] == code)
            assert np.array_equal(t[code]["local"][h, chans], np.arange(n))
        assert t[code]["width"] == max(int((lv[h] == code).sum()) for h in range(6))


# ---- quantize_key_page (layout.py:71-112) ---------------------------------------

def _kat_page():
    # heads=2, tokens=4, dim=4, levels LEVELS, one group of 4 tokens.
    page = np.zeros((2, 4, 4), F32)
    page[0, :, 0] = [0, 1, 2, 3]          # int2 -> codes 0,1,2,3 (s=1, lo=0)
    page[0, :, 3] = [3, 2, 1, 0]          # int2 -> codes 3,2,1,0
    page[0, :, 2] = [0, 15, 30, 45]       # int4 -> s=3, codes 0,5,10,15
    page[0, :, 1] = [0.5, -1.25, 2.0, 1024.0]  # fp16 tier
    page[1, :, 1] = [10, 11, 12, 13]      # int2 -> s=1, lo=10
    page[1, :, 2] = [-1, -1, -1, -1]      # int2 constant -> s=1e-5, codes 0
    page[1, :, 0] = [0, 255, 510, 765]    # int8 -> s=3, codes 0,85,170,255
    page[1, :, 3] = [0, 1, 2, 4]          # int4 -> s=4/15
    return page


def test_quantize_key_page_known_answer():
    table = layout.layer_table(LEVELS)
    out = layout.quantize_key_page(_kat_page(), table, 4)
    # tier 0: head0 slots (ch0, ch3), head1 slots (ch1, ch2); token-major words
    w0 = out[0]["code"].view(np.uint32)
    assert out[0]["code"].shape == (2, 4, 1)
    assert w0[0, :, 0].tolist() == [0 | 3 << 2, 1 | 2 << 2, 2 | 1 << 2, 3 | 0 << 2]
    assert w0[1, :, 0].tolist() == [0, 1, 2, 3]
    assert out[0]["scale"].shape == (2, 2, 1)
    assert out[0]["scale"].astype(F32)[:, :, 0].tolist() == [[1, 1], [1, np.float16(F32(1e-5)).item()]]
    assert out[0]["min"].astype(F32)[:, :, 0].tolist() == [[0, 0], [10, -1]]
    # tier 1: head0 ch2 (s=3), head1 ch3 (s=4/15)
    w1 = out[1]["code"].view(np.uint32)
    assert w1[0, :, 0].tolist() == [0, 5, 10, 15]
    # s = fp32(4/15) = 0.26666668 rounds up, so 2/s = 7.4999997 -> 7 (not 7.5 -> 8)
    assert w1[1, :, 0].tolist() == [0, 4, 7, 15]
    assert f16bits(out[1]["scale"][1, 0, 0]) == f16bits(np.float16(F32(4) / F32(15)))
    # tier 2: head0 has none -> padding scale 1, min 0, code 0; head1 ch0
    assert out[2]["code"].view(np.uint32)[0, :, 0].tolist() == [0, 0, 0, 0]
    assert out[2]["code"].view(np.uint32)[1, :, 0].tolist() == [0, 85, 170, 255]
    assert out[2]["scale"][0, 0, 0] == 1.0 and out[2]["min"][0, 0, 0] == 0.0
    assert out[2]["scale"][1, 0, 0] == 3.0
    # tier 3: head0 ch1 fp16 copies; head1 has none -> zero column
    assert out[3]["value"].shape == (2, 4, 1)
    assert out[3]["value"][0, :, 0].tolist() == [0.5, -1.25, 2.0, 1024.0]
    assert out[3]["value"][1, :, 0].tolist() == [0, 0, 0, 0]


def test_key_groups_run_along_tokens():
    table = layout.layer_table(np.zeros((1, 2), np.int64))
    page = np.zeros((1, 8, 2), F32)
    page[0, :4, 0] = [0, 1, 2, 3]
    page[0, 4:, 0] = [0, 10, 20, 30]
    page[0, :, 1] = np.arange(8)
    out = layout.quantize_key_page(page, table, 4)
    assert out[0]["scale"].shape == (1, 2, 2)                  # [heads, width, groups]
    assert out[0]["scale"].astype(F32)[0].tolist() == [[1, 10], [1, 1]]
    assert out[0]["min"].astype(F32)[0].tolist() == [[0, 0], [0, 4]]
    with pytest.raises(ValueError):
        layout.quantize_key_page(page, table, 3)


def test_value_page_known_answer():
    page = np.zeros((1, 2, 32), F32)
    page[0, 0, :16] = np.tile([0, 1, 2, 3], 4)
    page[0, 0, 16:] = np.tile([3, 2, 1, 0], 4)
    page[0, 1] = np.linspace(-1, 1, 32, dtype=F32)
    out = layout.quantize_value_page(page, 2, 16)
    assert out["code"].shape == (1, 2, 2) and out["scale"].shape == (1, 2, 2)
    w = out["code"].view(np.uint32)[0, 0]
    assert w[0] == sum(c << (2 * i) for i, c in enumerate([0, 1, 2, 3] * 4))
    assert w[1] == sum(c << (2 * i) for i, c in enumerate([3, 2, 1, 0] * 4))
    assert out["min"].astype(F32)[0, 1].tolist() == [-1.0, np.float16(page[0, 1, 16]).item()]
    assert layout.quantize_value_page(page, 16, 16)["value"].dtype == np.float16
    with pytest.raises(ValueError):
        layout.quantize_value_page(page, 2, 12)


# ---- dequantisation (layout.py:132-182) -----------------------------------------

def test_dequantize_known_answer_and_fp16_tier():
    table = layout.layer_table(LEVELS)
    out = layout.quantize_key_page(_kat_page(), table, 4)
    deq = layout.dequantize_key(4, table, out, 4)
    assert deq[0, :, 0].tolist() == [0, 1, 2, 3]
    assert deq[0, :, 2].tolist() == [0, 15, 30, 45]
    assert deq[0, :, 1].tolist() == [0.5, -1.25, 2.0, 1024.0]
    assert deq[1, :, 0].tolist() == [0, 255, 510, 765]
    assert np.all(deq[1, :, 2] == -1)


def test_roundtrip_error_bound():
    rng = np.random.default_rng(5)
    lv = rng.integers(0, 4, size=(4, 64))
    table = layout.layer_table(lv)
    page = (rng.standard_normal((4, 128, 64)) * rng.lognormal(0, 1, (4, 1, 64))).astype(F32)
    page = page.astype(np.float16).astype(F32)     # fp16-exact inputs keep the fp16 tier exact
    packed = layout.quantize_key_page(page, table, 128)
    deq = layout.dequantize_key(128, table, packed, 128)
    for code, bits in ((0, 2), (1, 4), (2, 8)):
        for h in range(4):
            n = int(table[code]["count"][h])
            ch = table[code]["index"][h, :n]
            x = page[h][:, ch]
            s16 = packed[code]["scale"][h, :n, 0].astype(F32)
            lo = x.min(0)
            s = (x.max(0) - lo) / F32((1 << bits) - 1)
            bound = s / 2 + ((1 << bits) - 1) * np.abs(s16 - s) + np.abs(packed[code]["min"][h, :n, 0] - lo) + 1e-5
            assert np.all(np.abs(deq[h][:, ch] - x) <= bound * 1.001)
    ch3 = lv == 3
    assert np.array_equal(deq[:, :, :][np.broadcast_to(ch3[:, None, :], deq.shape)],
                          page[np.broadcast_to(ch3[:, None, :], page.shape)])
    v = layout.quantize_value_page(page, 2, 64)
    dv = layout.dequantize_value(v, 128, 64, 2, 64)
    assert dv.shape == page.shape


def test_reference_test_pack_matches_group_quantizer():
    """Restates the reference's test_key_pack_matches_group_quantizer
    (tests/test_logitfill_offline.py:127-145): dequant(pack) ~ GroupQuantizer(2, 8)
    (quantizers/quantizer.py:25-41: restored = round((x + z)/s).clamp * s - z, z = -min,
    s, z kept in float32) along time for Key and along features for Value, atol=rtol=1e-2."""
    torch = pytest.importorskip("torch")
    torch.manual_seed(0)
    page = torch.randn(2, 16, 8).numpy()

    def group_quant(x, bits, group):            # last axis grouped
        flat = x.reshape(-1, group).astype(F32)
        mx, mn = flat.max(1, keepdims=True), flat.min(1, keepdims=True)
        s = np.clip((mx - mn) / F32((1 << bits) - 1), F32(1e-5), F32(1e5))
        z = -mn
        q = np.clip(np.rint((flat + z) / s), 0, (1 << bits) - 1)
        return (q * s - z).reshape(x.shape)

    table = layout.layer_table(np.zeros((2, 8), np.int64))
    packed = layout.quantize_key_page(page, table, 8)
    restored = layout.dequantize_key(16, table, packed, 8)
    ref = np.swapaxes(group_quant(np.swapaxes(page, 1, 2), 2, 8), 1, 2)
    assert np.allclose(restored, ref, atol=1e-2, rtol=1e-2)
    values = layout.quantize_value_page(page, 2, 8)
    restored_v = layout.dequantize_value(values, 16, 8, 2, 8)
    assert np.allclose(restored_v, group_quant(page, 2, 8), atol=1e-2, rtol=1e-2)
