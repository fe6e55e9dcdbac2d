"""Write ``packer_golden.npz``: input/output vectors of the reference packer.

Run in a container that holds the reference checkout (``LOGITFILL_REF``,
default ``/root/reference``)::

    python tests/golden/make_golden.py

It loads the reference's ``src/logitfill/packed/layout.py`` by file path (the
module imports only torch) and calls, on CPU, the functions the packed decode
path's page compress must match bit for bit:

* ``tier_tables`` (``layout.py:49-68``),
* ``quantize_key_page`` (``layout.py:71-112``) and ``quantize_value_page``
  (``layout.py:115-129``), page by page, with the pages concatenated along the
  reference history axes (``cache.py:64-81``: codes and fp16 values along
  tokens, Key scale/min along groups, Value scale/min along tokens).

The fixture stores, per case, the inputs (levels, Key and Value in their source
dtype's bits) and the outputs (int32 codes, fp16 scale/min/value bits).  Tests
read only the fixture; nothing at test time touches the reference.
"""
from __future__ import annotations

import importlib.util
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from logitfill_amd import synth  # noqa: E402

REF = Path(os.environ.get("LOGITFILL_REF", "/root/reference"))
OUT = HERE / "packer_golden.npz"


def load_reference_layout():
    path = REF / "src" / "logitfill" / "packed" / "layout.py"
    spec = importlib.util.spec_from_file_location("logitfill_reference_layout", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def cases():
    """(name, levels [n_kv, D] int64, key, value [n_kv, T, D] torch, page, k_group, v_group, bit_v)."""
    out = []
    # BASELINE config 0 (first page of layer 0 at seed 0), bf16
    d = synth.make_layer(1, 28, 4, 128, 128, 2.5, seed=0)
    out.append(("config0", d.levels, d.key[0], d.value[0], 128, 128, 128, 2))
    # two pages, fp16 source, target 3.0
    d = synth.make_layer(1, 8, 2, 128, 256, 3.0, seed=5, dtype=torch.float16)
    out.append(("fp16_two_pages", d.levels, d.key[0], d.value[0], 128, 128, 128, 2))
    # the reference's own CUDA-test shape (tests/test_logitfill_offline.py:198-213): D 64, page 64
    g = torch.Generator().manual_seed(0)
    levels = torch.randint(0, 4, (1, 64), generator=g)
    out.append(("reference_test_shape", levels.numpy(), torch.randn(1, 64, 64, generator=g),
                 torch.randn(1, 64, 64, generator=g), 64, 64, 64, 2))
    # Key-group / Value-group / Value-width variants
    for i, (kg, vg, bv) in enumerate([(64, 128, 2), (32, 64, 2), (128, 32, 4), (128, 16, 8), (128, 128, 16)]):
        d = synth.make_layer(1, 4, 1, 128, 128, 3.0, seed=100 + i)
        out.append((f"groups_k{kg}_v{vg}_b{bv}", d.levels, d.key[0], d.value[0], 128, kg, vg, bv))
    # edge values at the common shape (D 128, page = groups = 128)
    g = torch.Generator().manual_seed(7)
    D, T = 128, 128
    levels = np.tile(np.array([0, 1, 2, 3, 0, 0, 1, 0]), 16)[None].repeat(2, 0)
    key = torch.randn(2, T, D, generator=g) * 3
    key[0, :, 0] = 7.0                                        # constant group: s clamps to 1e-5
    key[0, :, 1] = torch.linspace(-3e5, 3e5, T)               # int4 range beyond fp16 max * 15
    key[0, :, 4] = torch.tensor([0.0, 0.5, 1.5, 2.5, 3.0] * 25 + [0.0, 0.0, 3.0])   # exact ties
    key[1, :, 0] = torch.randn(T, generator=g) * 1e-30        # tiny values
    key[1, :, 3] = torch.randn(T, generator=g) * 1e5          # fp16 tier overflows to +-inf
    key[1, :, 7] = -0.0
    key[1, 5, 8] = 3e38                                       # range overflows float32
    key[1, 6, 8] = -3e38
    key = key.bfloat16()
    value = (torch.randn(2, T, D, generator=g) * torch.logspace(-6, 6, D)).bfloat16()
    value[0, 3] = 1.0                                         # constant Value row
    value[1, 9, :64] = 2e38
    value[1, 9, 64:] = -2e38
    out.append(("edge_values", levels, key, value, 128, 128, 128, 2))
    # division-sensitive ties: (x - lo) / s is exactly k + 0.5 after IEEE division
    key = torch.zeros(1, 128, 128, dtype=torch.float32)
    for i, (sb, db) in enumerate([(1081804425, 1135190891), (1090252937, 1154556202), (1092564827, 1153771404)]):
        s = np.array([sb], np.uint32).view(np.float32)[0]
        dd = np.array([db], np.uint32).view(np.float32)[0]
        key[0, 1, i] = float(dd)
        key[0, 2, i] = float(np.float32(s * np.float32(255)))
    levels = np.full((1, 128), 2, np.int64)
    levels[0, 100:] = 0
    out.append(("division_ties", levels, key, key.clone(), 128, 128, 128, 2))
    return out


def bits(t: torch.Tensor) -> np.ndarray:
    """Raw bits of a tensor (2-byte dtypes as uint16, float32 as float32, ints as is)."""
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16)
    return t.contiguous().numpy()


def main() -> None:
    ref = load_reference_layout()
    arrays = {}
    names = []
    for name, levels, key, value, page, kg, vg, bv in cases():
        names.append(name)
        levels_t = torch.as_tensor(np.asarray(levels), dtype=torch.int64)
        built = ref.tier_tables(levels_t)
        table = built["tiers"]
        n_pages = key.shape[1] // page
        hk, hv = None, None
        for p in range(n_pages):
            kp = ref.quantize_key_page(key[:, p * page:(p + 1) * page], table, kg)
            vp = ref.quantize_value_page(value[:, p * page:(p + 1) * page], bv, vg)
            if hk is None:
                hk, hv = kp, vp
                continue
            for t in (0, 1, 2):
                hk[t]["code"] = torch.cat((hk[t]["code"], kp[t]["code"]), dim=1)
                hk[t]["scale"] = torch.cat((hk[t]["scale"], kp[t]["scale"]), dim=2)
                hk[t]["min"] = torch.cat((hk[t]["min"], kp[t]["min"]), dim=2)
            hk[3]["value"] = torch.cat((hk[3]["value"], kp[3]["value"]), dim=1)
            for k in hv:
                hv[k] = torch.cat((hv[k], vp[k]), dim=1)
        pre = name + "/"
        arrays[pre + "meta"] = np.array([page, kg, vg, bv, n_pages], np.int64)
        arrays[pre + "levels"] = np.asarray(levels, np.int64)
        arrays[pre + "src_dtype"] = np.array(str(key.dtype).replace("torch.", ""))
        arrays[pre + "key"] = bits(key)
        arrays[pre + "value"] = bits(value)
        for t in (0, 1, 2, 3):
            for k in ("index", "count", "local"):
                arrays[f"{pre}table{t}_{k}"] = table[t][k].numpy()
            arrays[f"{pre}table{t}_width"] = np.array(int(table[t]["width"]), np.int64)
        arrays[pre + "tier"] = built["tier"].numpy()
        for t in (0, 1, 2):
            arrays[f"{pre}k{t}_code"] = hk[t]["code"].numpy()
            arrays[f"{pre}k{t}_scale"] = bits(hk[t]["scale"])
            arrays[f"{pre}k{t}_min"] = bits(hk[t]["min"])
        arrays[pre + "k3_value"] = bits(hk[3]["value"])
        for k in hv:
            arrays[f"{pre}v_{k}"] = bits(hv[k])
    arrays["cases"] = np.array(names)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(names)} cases)")


if __name__ == "__main__":
    main()
