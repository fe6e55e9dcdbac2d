"""A tier-table policy on disk drives the packed cache end to end (reference adapter
``load_policy`` + ``packed_manager``, src/logitfill/models/deepseek_qwen.py:111-137), and the
stored bytes of a live cache layer equal the stored-layout footprint count."""
import numpy as np
import pytest
import torch

from logitfill_amd import footprint, policy, synth
from logitfill_amd.packed.reference import decode_into
from tests.helpers import assert_decode_close, f32, oracle_decode, oracle_store

pytestmark = pytest.mark.gpu


def test_policy_file_drives_decode(gpu, tmp_path):
    n_layers, n_kv, n_q, D = 2, 2, 8, 128
    levels = np.stack([synth.sample_tier_levels(n_kv, D, 3.0, seed=80 + s) for s in range(n_layers)])
    policy.build_policy(levels, model_id="test-model", target_bit=3.0).save(tmp_path / "pol")
    pol = policy.PrecisionPolicy.load(tmp_path / "pol")
    mgr = policy.manager_from_policy(pol, n_q, gpu, batch_size=1)
    with pytest.raises(ValueError):
        policy.manager_from_policy(pol, n_q, gpu, bit_v=4)
    T = 5 * 128 + 17
    for layer in range(n_layers):
        d = synth.make_layer(1, n_q, n_kv, D, T, 3.0, seed=90 + layer)
        d.levels = pol.levels[layer]
        mgr.commit(layer, d.key.to(gpu), d.value.to(gpu))
        q = d.query.to(gpu)
        out = torch.empty_like(q)
        decode_into(mgr, layer, q, d.key_new.to(gpu), d.value_new.to(gpu), D ** -0.5, out)
        torch.cuda.synchronize()
        store = oracle_store(d.levels, f32(d.key[0]), f32(d.value[0]))
        ref = oracle_decode(store, f32(d.query[0]), f32(d.key_new[0]), f32(d.value_new[0]), D ** -0.5, n_q, n_kv)
        assert_decode_close(out[0], ref)


@pytest.mark.parametrize("tb,tokens", [(2.5, 3 * 128 + 40), (3.0, 7 * 128)])
def test_stored_bytes_match_footprint(gpu, tb, tokens):
    n_kv, n_q, D = 4, 28, 128
    d = synth.make_layer(1, n_q, n_kv, D, tokens, tb, seed=11)
    from logitfill_amd.packed import PackedKVManager
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu)
    mgr.commit(0, d.key.to(gpu), d.value.to(gpu))
    live = footprint.stored_bytes(mgr.layers[0], 0)
    want = footprint.stored_footprint(d.levels[None], tokens)
    for key in ("k_payload_bytes", "v_payload_bytes", "scale_min_bytes", "residual_bytes", "page_copy_bytes"):
        assert live[key] == want[key], key
    assert live["history_tokens"] == want["history_tokens"] and live["residual_tokens"] == want["residual_tokens"]
