"""CPU tests of the host side: tier tables, sampler, the C ABI library's exports,
struct layouts against the C compiler, the host-only planner and argument
validation (no device work is enqueued by any call here)."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import layout as product_layout
from oracle import layout as oracle_layout

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "logitfill_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lf_[a-z0-9_]+)\s*\(", text)))


def test_product_tier_tables_match_oracle():
    rng = np.random.default_rng(0)
    for lv in [np.array([[0, 3, 1, 0], [2, 0, 0, 1]]), rng.integers(0, 4, (8, 128)),
               synth.sample_tier_levels(4, 128, 2.5, 3), np.zeros((2, 64), np.int64)]:
        ours = product_layout.tier_tables(torch.as_tensor(lv))
        ref = oracle_layout.tier_tables(lv)
        assert np.array_equal(ours["tier"].numpy(), ref["tier"])
        for t in range(4):
            for k in ("index", "count", "local"):
                assert np.array_equal(ours["tiers"][t][k].numpy(), ref["tiers"][t][k]), (t, k)
            assert ours["tiers"][t]["width"] == ref["tiers"][t]["width"]
    with pytest.raises(ValueError):
        product_layout.tier_tables(torch.tensor([[0, 4]]))


@pytest.mark.parametrize("target", [2.5, 3.0, 4.0])
def test_sampler_spends_exact_budget(target):
    lv = synth.sample_tier_levels(8, 128, target, seed=11)
    budget = synth.key_budget(target)
    assert np.all(synth.LEVEL_EXTRA[lv].sum(-1) == budget)
    assert synth.LEVEL_BITS[lv].mean() == 2 * target - 2
    assert np.array_equal(lv, synth.sample_tier_levels(8, 128, target, seed=11))


def test_budget_rule_matches_reference_selfcheck():
    # reference allocators/allocate.py:20-25 and :160-164
    assert synth.key_budget(2.5, 2, 128) == 128
    with pytest.raises(ValueError):
        synth.key_budget(1.5, 2, 128)


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = declared_functions()
    assert "lf_decode_attention" in names and "lf_pack_pages" in names
    for name in names:
        assert hasattr(lib, name), name
        assert name in _native._SIGNATURES, f"{name} has no ctypes signature"
    assert lib.lf_abi_version() == _native.ABI_VERSION == 8
    assert b"gfx950" in lib.lf_build_info()


def test_struct_layouts_match_c(tmp_path):
    fields = {
        "lf_packed_layer": [f for f, _ in _native.PackedLayer._fields_],
        "lf_decode_args": [f for f, _ in _native.DecodeArgs._fields_],
        "lf_pack_source": [f for f, _ in _native.PackSource._fields_],
    }
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for st, fs in fields.items():
        lines.append(f'printf("{st} %zu\\n", sizeof({st}));')
        for f in fs:
            lines.append(f'printf("{st}.{f} %zu\\n", offsetof({st}, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-o", str(exe), str(src)], check=True)
    out = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                               check=True).stdout.split("\n") if line)
    for st, cls in (("lf_packed_layer", _native.PackedLayer), ("lf_decode_args", _native.DecodeArgs),
                    ("lf_pack_source", _native.PackSource)):
        assert int(out[st]) == ctypes.sizeof(cls), st
        for f in fields[st]:
            assert int(out[f"{st}.{f}"]) == getattr(cls, f).offset, (st, f)


def test_plan_decode_known_answer():
    """Hand-derived plans: each sequence's work (residual + pages) cut into equal items, the
    residual in the first item (kind 2, or 1 when that item holds no page)."""
    lib = _native.load()
    hp = (ctypes.c_int32 * 3)(5, 0, 2)
    work = (ctypes.c_int32 * 40)()
    seq = (ctypes.c_int32 * 6)()
    n = lib.lf_plan_decode(hp, 3, 2, 1, work, 10, seq)
    assert n == 6
    items = np.array(list(work)[:24]).reshape(6, 4).tolist()
    assert items == [[0, 0, 1, 2], [0, 1, 3, 0], [0, 3, 5, 0],   # work 6 -> 3 items of 2
                     [1, 0, 0, 1],                               # no pages: residual only
                     [2, 0, 0, 1], [2, 0, 2, 0]]                 # work 3 -> items of 1 and 2
    assert list(seq) == [0, 3, 3, 1, 4, 2]
    n = lib.lf_plan_decode(hp, 3, 2, 0, work, 10, seq)
    assert n == 5
    assert np.array(list(work)[:20]).reshape(5, 4).tolist() == [
        [0, 0, 1, 2], [0, 1, 3, 0], [0, 3, 5, 0], [1, 0, 0, 1], [2, 0, 2, 2]]
    assert list(seq) == [0, 3, 3, 1, 4, 1]
    assert lib.lf_plan_decode(hp, 3, 2, 1, work, 5, seq) == -4       # LF_E_WORKSPACE
    assert lib.lf_plan_decode(hp, 3, 0, 1, work, 10, seq) == -2      # LF_E_SHAPE
    assert lib.lf_plan_decode(hp, 3, 2, -1, work, 10, seq) == -2     # LF_E_SHAPE


@pytest.mark.parametrize("pps,res", [(1, 0), (3, 5), (7, 2), (32, 5), (33, 5)])
def test_plan_decode_covers_pages(pps, res):
    """Every page of every sequence lies in exactly one item, in order; items of a sequence
    are consecutive; exactly its first item carries the residual; item work is balanced
    to within one page."""
    lib = _native.load()
    pages = [0, 1, 7, 64, 256, 257, 3]
    B = len(pages)
    hp = (ctypes.c_int32 * B)(*pages)
    cap = 4 * B + sum(pages)
    work = (ctypes.c_int32 * (4 * cap))()
    seq = (ctypes.c_int32 * (2 * B))()
    n = lib.lf_plan_decode(hp, B, pps, res, work, cap, seq)
    assert n > 0
    items = np.array(list(work)[: 4 * n]).reshape(n, 4)
    for b in range(B):
        first, count = seq[2 * b], seq[2 * b + 1]
        it = items[first:first + count]
        assert (it[:, 0] == b).all()
        assert it[0, 3] in (1, 2) and (it[1:, 3] == 0).all()
        covered = np.concatenate([np.arange(p0, p1) for _, p0, p1, _ in it])
        assert covered.tolist() == list(range(pages[b]))
        if pages[b]:
            assert count == -(-(pages[b] + res) // pps) or (it[:, 2] > it[:, 1]).sum() < count
            w = (it[:, 2] - it[:, 1]) + np.where(it[:, 3] > 0, res, 0)
            assert w.max() - w.min() <= 1 or res > w.min()
    assert sum(seq[2 * b + 1] for b in range(B)) == n


def test_workspace_layout():
    """Workspace = fp32 partials (o[D], m, l) per item and q head; bad shapes are rejected."""
    lib = _native.load()
    assert lib.lf_decode_workspace_bytes(28, 128, 100) == 100 * 28 * 130 * 4
    assert lib.lf_decode_workspace_bytes(28, 128, 1) == 28 * 130 * 4
    assert lib.lf_decode_workspace_bytes(0, 128, 1) == -2


def test_argument_validation_rejects_before_launch():
    lib = _native.load()
    assert lib.lf_pack_pages(None, None, None, 0, 0, 0, 0, None, 1, None) == -1
    layer = _native.PackedLayer()
    assert lib.lf_pack_pages(layer, None, None, 0, 0, 0, 0, None, 1, None) == -2   # zero shapes
    assert lib.lf_decode_attention(layer, None, None) == -2
    assert lib.lf_dequantize(layer, 0, 4, None, None, None) == -1
    assert lib.lf_dense_decode(None, None, None, 1, 1, 1, 128, 1, 0, 0, 0, 1.0, None, 64, None, 0, None) == -1
    # more than 2^21 page jobs in one call is refused
    assert lib.lf_pack_pages_multi(None, None, None, None, 1, 0, None, (1 << 21) + 1, None) == -2
    assert lib.lf_pack_pages_multi(None, None, None, None, 1, 0, None, 1 << 21, None) == -1


def test_layout_helper_validation_rejects_before_launch():
    """The device layout helpers check sizes on the host; nothing is launched here."""
    lib = _native.load()
    assert lib.lf_pack_ints(None, 1, 4, 33, None, None) == -2         # wider than a word
    assert lib.lf_pack_ints(None, 1, 4, 0, None, None) == -2
    assert lib.lf_pack_ints(None, 1, 4, 3, None, None) == -1          # 3 bits: ten slots a word
    assert lib.lf_unpack_ints(None, 1, 1, 11, 3, None, None) == -2    # 11 slots > 1 word x 10
    assert lib.lf_unpack_ints(None, 1, 1, 2, 32, None, None) == -2    # bits 32: one slot a word
    assert lib.lf_pack_ints(None, 0, 4, 2, None, None) == 0           # empty: nothing to do
    assert lib.lf_pack_ints(None, 1, 4, 2, None, None) == -1
    assert lib.lf_unpack_ints(None, 1, 1, 17, 2, None, None) == -2    # 17 slots > 1 word x 16
    assert lib.lf_unpack_ints(None, 1, 1, 16, 2, None, None) == -1
    assert lib.lf_asymmetric_codes(None, 7, 1, 4, 2, None, None, None, None) == -5
    assert lib.lf_asymmetric_codes(None, 0, 1, 4, 0, None, None, None, None) == -2
    assert lib.lf_asymmetric_codes(None, 0, 0, 4, 2, None, None, None, None) == 0


def test_padded_value_words_accepted():
    """Value rows whose width is not a word multiple are padded (reference layout.py:27-29),
    and the layer check wants ceil(head_dim * bit_v / 32) words: a D 8 int2 layer has one."""
    from logitfill_amd.packed.layout import value_words

    assert value_words(8, 2) == 1 and value_words(128, 2) == 8 and value_words(24, 4) == 3
    assert value_words(100, 8) == 25 and value_words(12, 8) == 3


def test_decode_commit_arguments_rejected_before_launch():
    """lf_decode_args.commit_new: only 0 or 1, and 1 needs the new rows and room for them in the
    tail; each of these calls returns LF_E_SHAPE from the host checks, before anything touches
    a device (the pointers are placeholders that are never dereferenced)."""
    lib = _native.load()
    fake = 0x1000
    L = _native.PackedLayer()
    L.batch, L.n_kv, L.head_dim, L.page_size, L.k_group = 2, 4, 128, 128, 128
    L.cap_tokens, L.cap_kgroups = 1024, 8
    L.k_width[:] = [64, 32, 32, 0]
    L.k_words[:] = [4, 4, 8]
    for t in range(3):
        L.k_code[t] = L.k_scale[t] = L.k_min[t] = fake
        L.tier_index[t] = L.tier_count[t] = fake
    L.bit_v, L.v_group, L.v_groups, L.v_words = 2, 128, 1, 8
    L.v_code = L.v_scale = L.v_min = fake
    a = _native.DecodeArgs()
    a.query = a.out = a.work = a.seq_work = a.tail_len = fake
    a.k_new = a.v_new = a.tail_k = a.tail_v = fake
    a.q_dtype = a.out_dtype = a.tail_dtype = a.new_dtype = _native.LF_BF16
    a.n_q, a.q_len, a.n_work, a.tail_cap, a.scaling = 28, 1, 4, 128, 1.0
    a.workspace, a.workspace_bytes = fake, 1 << 30
    a.commit_new = 2
    assert lib.lf_decode_attention(L, a, None) == -2
    a.commit_new, a.tail_cap = 1, 0
    assert lib.lf_decode_attention(L, a, None) == -2          # no tail rows to append into
    a.tail_cap, a.q_len = 128, 200
    assert lib.lf_decode_attention(L, a, None) == -2          # more new rows than the tail holds
    a.q_len, a.k_new, a.v_new = 1, 0, 0
    assert lib.lf_decode_attention(L, a, None) == -2          # nothing to append
