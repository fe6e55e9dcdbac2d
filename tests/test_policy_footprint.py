"""Tier-table policy files (reference src/logitfill/allocators/policy.py:28-128 and the
budget rule of allocate.py:14-88,138-147) and footprint accounting (memory.py:14-98, plus
the stored-layout count), on the CPU.  Known answers are worked by hand in the comments."""
import json
from types import SimpleNamespace

import numpy as np
import pytest

import bench
from logitfill_amd import footprint, policy, synth


def _levels(n_layers=3, n_kv=2, D=128, tb=2.5):
    return np.stack([synth.sample_tier_levels(n_kv, D, tb, seed=s) for s in range(n_layers)])


def test_budget_known_answers():
    # target_bit_k = 2 * target_bit - bit_v; extra = round((target_bit_k - 2) * channels)
    b = policy.kv_history_budget(2.5)
    assert (b["target_bit_k"], b["extra_budget_per_head"]) == (3.0, 128)
    assert policy.kv_history_budget(3.0)["extra_budget_per_head"] == 256
    assert policy.kv_history_budget(3.0, bit_v=4)["extra_budget_per_head"] == 0  # Key target 2.0
    assert policy.kv_history_budget(2.5, n_channels=64)["extra_budget_per_head"] == 64
    with pytest.raises(ValueError):
        policy.kv_history_budget(1.5)  # Key target 1.0 < int2 floor
    with pytest.raises(ValueError):
        policy.kv_history_budget(2.5, bit_v=1)
    # one head: 3 int4 (2 bits each above int2), 1 int8 (6), 1 fp16 (14) -> 26 extra bits
    lv = np.zeros((1, 16), dtype=np.int64)
    lv[0, :3] = 1
    lv[0, 3] = 2
    lv[0, 4] = 3
    assert int(policy.spent_extra_per_head(lv)[0]) == 26
    h = policy.level_histogram(lv)
    assert (h["int2"], h["int4"], h["int8"], h["fp16"]) == (11.0, 3.0, 1.0, 1.0)
    assert h["actual_bit_k"] == pytest.approx((11 * 2 + 3 * 4 + 8 + 16) / 16)


def test_policy_roundtrip_and_metadata(tmp_path):
    lv = _levels()
    curves = {"d2": np.random.default_rng(0).random(lv.shape)}
    pol = policy.build_policy(lv, model_id="models/DeepSeek-R1-Distill-Qwen-7B", target_bit=2.5, curves=curves)
    meta = pol.metadata
    assert (meta["n_layers"], meta["n_kv"], meta["head_dim"]) == (3, 2, 128)
    assert (meta["target_bit_k"], meta["extra_budget_per_head"]) == (3.0, 128)
    assert meta["achieved"]["actual_bit_k"] == pytest.approx(3.0)  # the sampler spends the budget exactly
    pol.save(tmp_path / "p")
    assert json.loads((tmp_path / "p" / "metadata.json").read_text()) == json.loads(json.dumps(meta))
    back = policy.PrecisionPolicy.load(tmp_path / "p")
    assert np.array_equal(back.levels, lv) and back.levels.dtype == np.int64
    assert set(back.curves) == {"d2"} and np.array_equal(back.curves["d2"], curves["d2"])
    assert back.metadata == json.loads(json.dumps(meta))


def test_policy_rejects_bad_inputs():
    lv = _levels()
    meta = {"target_bit": 2.5, "n_layers": 3, "n_kv": 2, "head_dim": 128}
    policy.PrecisionPolicy(lv, meta)
    with pytest.raises(ValueError):
        policy.PrecisionPolicy(lv[0], meta)  # not 3-D
    bad = lv.copy()
    bad[0, 0, 0] = 4
    with pytest.raises(ValueError):
        policy.PrecisionPolicy(bad, {})
    with pytest.raises(ValueError):
        policy.PrecisionPolicy(lv, dict(meta, n_kv=4))
    over = lv.copy()
    over[1, 0, :] = 1  # 128 channels at int4: 256 extra bits > 128
    with pytest.raises(ValueError):
        policy.PrecisionPolicy(over, meta)
    policy.PrecisionPolicy(over, dict(meta, enforce_budget=False))
    with pytest.raises(ValueError):
        policy.PrecisionPolicy(lv, meta, {"c": np.zeros((3, 2, 64))})


def test_validate_model():
    pol = policy.build_policy(_levels(), model_id="deepseek-ai/DeepSeek-R1-Distill-Qwen-7B", target_bit=2.5)
    cfg = SimpleNamespace(num_hidden_layers=3, num_key_value_heads=2, num_attention_heads=14, hidden_size=1792,
                          name_or_path="/models/DeepSeek-R1-Distill-Qwen-7B")
    pol.validate_model(SimpleNamespace(config=cfg))  # head_dim from hidden_size // heads; same basename
    with pytest.raises(ValueError):
        pol.validate_model(SimpleNamespace(config=SimpleNamespace(**dict(vars(cfg), num_key_value_heads=4))))
    with pytest.raises(ValueError):
        pol.validate_model(SimpleNamespace(config=SimpleNamespace(**dict(vars(cfg), name_or_path="Qwen2-7B"))))


def _small_levels():
    # head 0: 20 int2, 8 int4, 2 int8, 2 fp16; head 1: 16 int2, 12 int4, 4 int8
    h0 = [0] * 20 + [1] * 8 + [2] * 2 + [3] * 2
    h1 = [0] * 16 + [1] * 12 + [2] * 4
    return np.array([[h0, h1]], dtype=np.int64)


def test_runtime_footprint_known_answer():
    f = footprint.runtime_footprint(_small_levels(), 2 * 64 + 10, page_size=64, k_group_size=64, v_group_size=32)
    # hist 128, residual 10, groups 2
    assert f["k_payload_bytes"] == 128 * (120 + 112) / 8          # Key bits per token: 120 + 112
    assert f["v_payload_bytes"] == 128 * 2 * 64 / 8
    assert f["packing_padding_bytes"] == (12 + 4 + 2) * 128 / 8    # per-head word padding
    assert f["metadata_bytes"] == 62 * 2 * 4 + 128 * 2 * 1 * 4 + 64 * 2  # K scale/min, V scale/min, index
    assert f["residual_bytes"] == 10 * 64 * 4
    assert f["total_bytes"] == 10256
    assert f["effective_bit"] == pytest.approx(10256 * 8 / (138 * 64 * 2))


def test_stored_footprint_known_answer():
    f = footprint.stored_footprint(_small_levels(), 2 * 64 + 10, page_size=64, k_group_size=64, v_group_size=32)
    # widths (max over heads): int2 20 -> 2 words, int4 12 -> 2, int8 4 -> 1, fp16 2
    assert f["k_payload_bytes"] == 128 * 2 * 4 * 5 + 128 * 2 * 2 * 2
    assert f["scale_min_bytes"] == 2 * (20 + 12 + 4) * 2 * 4 + 128 * 2 * 1 * 4
    assert f["v_payload_bytes"] == 128 * 2 * 2 * 4
    assert f["table_bytes"] == 4 * (106 + 90 + 74 + 70) + 4 * 64
    assert f["residual_bytes"] == 10 * 64 * 4
    # page-major Key scale/min copy: int2 2 words -> 2 K-steps, int4 2 -> 1, int8 1 -> 1: 4 steps
    # of 4 blocks, 32 bytes a block, per page (2) and head (2)
    assert f["page_copy_bytes"] == 2 * 2 * 4 * 4 * 32
    assert f["total_bytes"] == sum(f[k] for k in ("k_payload_bytes", "v_payload_bytes", "metadata_bytes",
                                                  "residual_bytes", "page_copy_bytes"))


@pytest.mark.parametrize("tb", [2.5, 3.0])
def test_stored_footprint_is_what_decode_reads(tb):
    """bench.algorithmic_bytes (the roofline's numerator) counts exactly the stored history
    bytes, and the reference's analytical count understates them (cross-head padding)."""
    lv = _levels(n_layers=1, n_kv=4, tb=tb)
    H = 256 * 128
    st = footprint.stored_footprint(lv, H + 100)
    an = footprint.runtime_footprint(lv, H + 100)
    widths = [int((lv[0] == c).sum(-1).max()) for c in range(4)]
    words = [-(-widths[0] // 16), -(-widths[1] // 8), -(-widths[2] // 4)]
    total, _ = bench.algorithmic_bytes(widths, words, 4, 28, 128, H, 0)
    q_o = 4 * 28 * 128
    assert total - q_o == st["k_payload_bytes"] + st["v_payload_bytes"] + st["scale_min_bytes"]
    assert st["total_bytes"] - st["table_bytes"] > an["total_bytes"] - 4 * 128 * 2
