"""Parity at the BASELINE configurations the bench times, against the oracle.

* c1 (DeepSeek-R1-Distill-Qwen-1.5B shape): 12 q / 2 kv heads (GQA 6), batch 8, 64 packed
  pages + 37 residual tokens + the new token, target 2.5 -- the only GQA-6 shape, so the MFMA
  kernel's two padding head slots are exercised -- with the automatic kernel choice (MFMA)
  and the general VALU kernel;
* c2 at target 3.0 (Key 4.0 bits) at its own shape: 16 x (256 pages + 100 residual);
* c3 (page compress): one ``lf_pack_pages_multi`` launch over 28 layers x 64 sequences x 4 kv
  heads, at targets 2.5, 3.0 and 4.0 (Key 3.0, 4.0 and 6.0 bits), compared bit for bit with
  the oracle's packer (reference src/logitfill/packed/layout.py:71-129) on a subset of layers
  and sequences.

Decode outputs meet the north-star bar (max-abs 2e-3 or one bf16 ulp, rel-L2 1e-3) against
the oracle's dense dequantise-then-attend path (reference.py:30-56) over the device history
exported in the reference layout."""
import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from tests.helpers import assert_decode_close, assert_history_equal, f32, oracle_store
from tests.test_gpu_fullsize import _build, _decode, _oracle

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kernel", [_native.KERNEL_AUTO, _native.KERNEL_VALU])
def test_config1_shape(gpu, kernel):
    B, n_q, n_kv = 8, 12, 2
    d, mgr = _build(gpu, B, n_q, n_kv, [64] * B, [37] * B, 2.5, seed=21)
    scaling = 128 ** -0.5
    q = d.query
    out = torch.empty_like(q)
    from logitfill_amd.packed.reference import decode_into

    decode_into(mgr, 0, q, d.key_new, d.value_new, scaling, out, kernel=kernel)
    torch.cuda.synchronize()
    for b in (0, 5, 7):
        print(f"c1 shape: kernel {kernel}, sequence {b}", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))


def test_config2_target_3_at_its_shape(gpu):
    B, n_q, n_kv = 16, 28, 4
    d, mgr = _build(gpu, B, n_q, n_kv, [256] * B, [100] * B, 3.0, seed=22)
    assert mgr.layers[0].words[0] < 8  # Key 4.0 bits: fewer int2 words than at target 2.5
    scaling = 128 ** -0.5
    out = _decode(d, mgr, gpu, scaling)
    for b in (0, 11):
        print(f"c2 target 3.0: sequence {b}", flush=True)
        assert_decode_close(out[b], _oracle(d, mgr, b, n_q, n_kv, scaling))


@pytest.mark.parametrize("target", [2.5, 3.0, 4.0])
def test_config3_one_launch_pack_bit_exact(gpu, target):
    """The bench's config-3 pass (one launch for all layers' pages) against the oracle packer."""
    B, n_kv, D, L = 64, 4, 128, 28
    levels = [synth.sample_tier_levels(n_kv, D, target, seed=layer) for layer in range(L)]
    mgr = PackedKVManager(levels, 28, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B, capacity_tokens=128)
    srcs = []
    for layer in range(L):
        d = synth.make_layer(B, 28, n_kv, D, 128, target, seed=layer)
        srcs.append((d.key, d.value))
        mgr.layers[layer].reserve(128)
    dev_srcs = [(k.to(gpu), v.to(gpu)) for k, v in srcs]
    structs = (_native.PackedLayer * L)(*[mgr.layers[i].layer_struct() for i in range(L)])
    ps = (_native.PackSource * L)(*[_native.PackSource(k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
                                                       k.stride(2)) for k, v in dev_srcs])
    ds = torch.frombuffer(bytearray(structs), dtype=torch.uint8).to(gpu)
    dp = torch.frombuffer(bytearray(ps), dtype=torch.uint8).to(gpu)
    jobs = torch.tensor([(i, b, 0, 0) for i in range(L) for b in range(B)], dtype=torch.int32).to(gpu)
    st = _native.load().lf_pack_pages_multi(ds.data_ptr(), structs, dp.data_ptr(), ps, L, _native.LF_BF16,
                                            jobs.data_ptr(), L * B, _native.current_stream_ptr(gpu))
    _native.check(st, "lf_pack_pages_multi")
    torch.cuda.synchronize()
    assert mgr.layers[0].words[2] >= 1 and (target < 4.0 or mgr.layers[0].widths[3] > 0)
    for layer in (0, 13, 27):
        lay = mgr.layers[layer]
        lay.hist_lens = [128] * B
        k, v = srcs[layer]
        for b in (0, 31, 63):
            print(f"c3 target {target}: layer {layer}, sequence {b}", flush=True)
            store = oracle_store(levels[layer], f32(k[b]), f32(v[b]))
            assert_history_equal(lay, b, store, tail=False)
