"""Golden vectors of the reference packer (``tests/golden/packer_golden.npz``,
written by ``tests/golden/make_golden.py`` from the reference's
``src/logitfill/packed/layout.py:49-129`` on CPU, pages concatenated along the
history axes of ``cache.py:64-81``).

The CPU tests pin the numpy oracle to those vectors bit for bit; the GPU test
runs the same inputs through the HIP page-compress kernel (``lf_pack_pages``,
via ``PackedKVManager.commit``) and demands the same bits.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import history as ohist
from oracle import layout as ol

GOLDEN = Path(__file__).resolve().parent / "golden" / "packer_golden.npz"


def _load():
    z = np.load(GOLDEN, allow_pickle=False)
    return {k: z[k] for k in z.files}


DATA = _load()
CASES = [str(c) for c in DATA["cases"]]


def _case(name):
    pre = name + "/"
    page, kg, vg, bv, n_pages = (int(x) for x in DATA[pre + "meta"])
    dtype = str(DATA[pre + "src_dtype"])
    return pre, page, kg, vg, bv, n_pages, dtype


def _source(pre, dtype):
    """Key and Value as torch tensors of the source dtype, ``[n_kv, T, D]``."""
    out = []
    for name in ("key", "value"):
        raw = DATA[pre + name]
        if dtype in ("bfloat16", "float16"):
            t = torch.from_numpy(raw.view(np.int16).copy()).view(getattr(torch, dtype))
        else:
            t = torch.from_numpy(raw.copy())
        out.append(t)
    return out


def _assert_same_bits(ours, ref, what):
    ours = np.ascontiguousarray(ours)
    ref = np.ascontiguousarray(ref)
    assert ours.shape == ref.shape, (what, ours.shape, ref.shape)
    assert ours.dtype.itemsize == ref.dtype.itemsize, (what, ours.dtype, ref.dtype)
    assert np.array_equal(ours.view(np.uint8), ref.view(np.uint8)), what


def _check_history(pre, hist_k, hist_v, bv, as_np):
    for t in (0, 1, 2):
        _assert_same_bits(as_np(hist_k[t]["code"]), DATA[f"{pre}k{t}_code"], (pre, t, "code"))
        _assert_same_bits(as_np(hist_k[t]["scale"]), DATA[f"{pre}k{t}_scale"], (pre, t, "scale"))
        _assert_same_bits(as_np(hist_k[t]["min"]), DATA[f"{pre}k{t}_min"], (pre, t, "min"))
    _assert_same_bits(as_np(hist_k[3]["value"]), DATA[pre + "k3_value"], (pre, "fp16 tier"))
    names = ("value",) if bv >= 16 else ("code", "scale", "min")
    for n in names:
        _assert_same_bits(as_np(hist_v[n]), DATA[f"{pre}v_{n}"], (pre, "value", n))


def test_fixture_covers_the_reference_test_shape_and_edges():
    assert {"config0", "reference_test_shape", "edge_values", "division_ties"} <= set(CASES)


@pytest.mark.parametrize("name", CASES)
def test_oracle_tier_tables_match_golden(name):
    pre = name + "/"
    built = ol.tier_tables(DATA[pre + "levels"])
    for t in (0, 1, 2, 3):
        for k in ("index", "count", "local"):
            assert np.array_equal(built["tiers"][t][k], DATA[f"{pre}table{t}_{k}"]), (name, t, k)
        assert built["tiers"][t]["width"] == int(DATA[f"{pre}table{t}_width"])
    assert np.array_equal(built["tier"], DATA[pre + "tier"])


@pytest.mark.parametrize("name", CASES)
def test_oracle_packer_matches_golden(name):
    pre, page, kg, vg, bv, n_pages, dtype = _case(name)
    key, value = _source(pre, dtype)
    store = ohist.pack_history(DATA[pre + "levels"], key.float().numpy(), value.float().numpy(),
                               page, kg, vg, bv)
    assert store.hist_len == page * n_pages
    _check_history(pre, store.hist_k, store.hist_v, bv, np.asarray)


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_gpu_packer_matches_golden(gpu, name):
    from logitfill_amd.packed import PackedKVManager

    pre, page, kg, vg, bv, n_pages, dtype = _case(name)
    key, value = _source(pre, dtype)
    levels = torch.from_numpy(DATA[pre + "levels"].copy())
    n_kv, _, dim = key.shape
    print(f"golden case {name}: n_kv {n_kv} D {dim} pages {n_pages} kg {kg} vg {vg} bit_v {bv} {dtype}",
          flush=True)
    mgr = PackedKVManager([levels], n_kv, n_kv, dim, page, kg, vg, bv, gpu)
    mgr.commit(0, key[None].to(gpu), value[None].to(gpu))
    torch.cuda.synchronize()
    layer = mgr.layers[0]
    assert layer.hist_lens[0] == page * n_pages
    hk, hv = layer.export_reference(0)
    _check_history(pre, hk, hv, bv, lambda t: t.cpu().numpy())
