"""Model-level Key precision policies: the tier table on disk.

A policy is one ``[n_layers, n_kv, head_dim]`` level map (0 = int2, 1 = int4,
2 = int8, 3 = fp16) shared by every request, plus the calibration metadata and
optional per-channel curves.  Same file format and checks as the reference's
``PrecisionPolicy`` (``src/logitfill/allocators/policy.py:28-86``,
``build_policy`` ``:89-128``) and the budget rule it enforces
(``src/logitfill/allocators/allocate.py:14-88,138-147``):

* ``policy.npz``: ``levels`` int64 plus one array per curve, all the levels'
  shape (``numpy.savez_compressed``; loaded with ``allow_pickle=False``);
* ``metadata.json``: the dictionary of ``build_policy`` (sorted keys, indent 2).

``manager_from_policy`` builds the packed cache that consumes the policy, the
role of the reference adapter's ``load_policy`` + ``packed_manager``
(``src/logitfill/models/deepseek_qwen.py:111-137``).
"""
from __future__ import annotations

import json
from datetime import datetime, timezone
from pathlib import Path

import numpy as np

from logitfill_amd import __version__

POLICY_VERSION = 1
LEVEL_BITS = np.array([2, 4, 8, 16], dtype=np.int64)
LEVEL_EXTRA = np.array([0, 2, 6, 14], dtype=np.int64)  # payload bits above the int2 floor


# ---- the budget rule (allocate.py:14-88) ----------------------------------------------------

def extra_budget_per_head(target_bit_k: float, n_channels: int = 128) -> int:
    """Integer Key bits per head above the int2 floor: ``round((target_bit_k - 2) * n)``."""
    spare = (float(target_bit_k) - 2.0) * n_channels
    if spare < 0:
        raise ValueError(f"target_bit_k {target_bit_k} is below the int2 floor")
    return int(round(spare))


def kv_history_budget(target_bit: float, bit_v: int = 2, n_channels: int = 128) -> dict:
    """Per-head Key budget of a K+V history target: ``target_bit_k = 2 * target_bit - bit_v``
    (the Value width is fixed; residual pages and scale/min metadata are outside the budget)."""
    if int(bit_v) < 2 or int(bit_v) > 16:
        raise ValueError(f"bit_v must be in 2..16, got {bit_v}")
    target_k = 2.0 * float(target_bit) - float(bit_v)
    if target_k < 2.0 or target_k > 16.0:
        raise ValueError(f"target_bit {target_bit} with bit_v {bit_v} implies Key target {target_k}, outside [2, 16]")
    return {"target_bit": float(target_bit), "bit_v": int(bit_v), "target_bit_k": float(target_k),
            "extra_budget_per_head": extra_budget_per_head(target_k, n_channels), "n_channels": int(n_channels)}


def _checked_levels(levels) -> np.ndarray:
    values = np.asarray(levels, dtype=np.int64)
    if np.any((values < 0) | (values > 3)):
        raise ValueError("levels must be in {0, 1, 2, 3}")
    return values


def spent_extra_per_head(levels) -> np.ndarray:
    """Extra Key bits above int2 of each head of a ``[..., head_dim]`` level map."""
    return LEVEL_EXTRA[_checked_levels(levels)].sum(axis=-1)


def achieved_history_bits(levels, bit_v: int = 2) -> dict:
    """Mean Key, Value and joint payload bits of a level map."""
    values = _checked_levels(levels)
    bit_k = float(LEVEL_BITS[values].mean()) if values.size else float("nan")
    return {"actual_bit_k": bit_k, "bit_v": float(bit_v), "actual_bit_kv": 0.5 * (bit_k + float(bit_v))}


def assert_history_budget(levels, target_bit: float, bit_v: int = 2) -> dict:
    """Raise when some head spends more extra bits than the per-head budget; else the budget
    dictionary with the largest spend and the achieved bits."""
    values = _checked_levels(levels)
    budget = kv_history_budget(target_bit, bit_v, int(values.shape[-1]))
    spent = spent_extra_per_head(values)
    most = int(spent.max()) if spent.size else 0
    if most > budget["extra_budget_per_head"]:
        raise ValueError(f"a head spends {most} extra Key bits, the budget is {budget['extra_budget_per_head']}")
    budget["extra_spent_per_head"] = most
    budget.update(achieved_history_bits(values, bit_v))
    return budget


def level_histogram(levels) -> dict:
    """Channels per head at each level, and the mean Key bits (``allocate.py:138-147``)."""
    values = np.asarray(levels)
    flat = values.reshape(-1)
    heads = int(np.prod(values.shape[:-1]))
    return {"fp16": float((flat == 3).sum() / heads), "int8": float((flat == 2).sum() / heads),
            "int4": float((flat == 1).sum() / heads), "int2": float((flat == 0).sum() / heads),
            "actual_bit_k": float(LEVEL_BITS[flat].mean()) if flat.size else float("nan")}


# ---- the policy ------------------------------------------------------------------------------

_AXIS = {"n_layers": 0, "n_kv": 1, "head_dim": 2}


class PrecisionPolicy:
    """Fixed per-channel Key levels ``[n_layers, n_kv, head_dim]`` plus calibration metadata."""

    def __init__(self, levels, metadata: dict, curves: dict | None = None):
        self.levels = np.asarray(levels, dtype=np.int64)
        if self.levels.ndim != 3:
            raise ValueError(f"levels must be [layers, kv_heads, head_dim], got {self.levels.shape}")
        if np.any((self.levels < 0) | (self.levels > 3)):
            raise ValueError("levels must be in {0, 1, 2, 3}")
        self.metadata = dict(metadata)
        self.curves = {name: np.asarray(value) for name, value in (curves or {}).items()}
        self._check_consistency()

    def _check_consistency(self) -> None:
        for key, axis in _AXIS.items():
            if key in self.metadata and int(self.metadata[key]) != self.levels.shape[axis]:
                raise ValueError(f"metadata {key}={self.metadata[key]} does not match levels {self.levels.shape}")
        if self.metadata.get("enforce_budget", True) and "target_bit" in self.metadata:
            assert_history_budget(self.levels, float(self.metadata["target_bit"]), int(self.metadata.get("bit_v", 2)))
        for name, curve in self.curves.items():
            if curve.shape != self.levels.shape:
                raise ValueError(f"curve {name} has shape {curve.shape}, levels are {self.levels.shape}")

    def validate_model(self, model) -> None:
        """Raise when a model (or its ``config``) cannot consume this policy: shape
        ``(num_hidden_layers, num_key_value_heads, head_dim)`` and, when both are known, the
        model id (compared by its last path component)."""
        config = getattr(model, "config", model)
        n_layers = int(config.num_hidden_layers)
        n_kv = int(config.num_key_value_heads)
        n_q = int(config.num_attention_heads)
        head_dim = int(getattr(config, "head_dim", None) or config.hidden_size // n_q)
        if tuple(self.levels.shape) != (n_layers, n_kv, head_dim):
            raise ValueError(f"policy shape {self.levels.shape} does not match model {(n_layers, n_kv, head_dim)}")
        model_id = getattr(config, "name_or_path", None) or getattr(config, "_name_or_path", None)
        saved = self.metadata.get("model_id")
        if saved and model_id and Path(str(saved)).name != Path(str(model_id)).name and str(saved) != str(model_id):
            raise ValueError(f"policy model_id {saved} does not match loaded model {model_id}")

    def save(self, directory) -> Path:
        path = Path(directory)
        path.mkdir(parents=True, exist_ok=True)
        np.savez_compressed(path / "policy.npz", levels=self.levels, **self.curves)
        (path / "metadata.json").write_text(json.dumps(self.metadata, indent=2, sort_keys=True) + "\n",
                                            encoding="utf-8")
        return path

    @classmethod
    def load(cls, directory) -> "PrecisionPolicy":
        path = Path(directory)
        with np.load(path / "policy.npz", allow_pickle=False) as packed:
            arrays = {name: packed[name] for name in packed.files}
        metadata = json.loads((path / "metadata.json").read_text(encoding="utf-8"))
        levels = arrays.pop("levels")
        return cls(levels, metadata, arrays)


def build_policy(levels, *, model_id: str, target_bit: float, bit_v: int = 2, k_group_size: int = 128,
                 v_group_size: int = 128, page_size: int = 128, calibration_datasets=None, n_samples: int = 0,
                 curves: dict | None = None, normalized: bool = True) -> PrecisionPolicy:
    """A checked policy from an allocator's level map, with the reference's metadata keys."""
    values = np.asarray(levels, dtype=np.int64)
    budget = assert_history_budget(values, target_bit, bit_v)
    metadata = {
        "policy_version": POLICY_VERSION,
        "code_version": __version__,
        "model_id": model_id,
        "n_layers": int(values.shape[0]),
        "n_kv": int(values.shape[1]),
        "head_dim": int(values.shape[2]),
        "k_group_size": int(k_group_size),
        "v_group_size": int(v_group_size),
        "page_size": int(page_size),
        "bit_v": int(bit_v),
        "target_bit": float(target_bit),
        "target_bit_k": budget["target_bit_k"],
        "extra_budget_per_head": budget["extra_budget_per_head"],
        "calibration_datasets": list(calibration_datasets or []),
        "n_samples": int(n_samples),
        "normalized": bool(normalized),
        "histogram": level_histogram(values),
        "achieved": achieved_history_bits(values, bit_v),
        "created_utc": datetime.now(timezone.utc).isoformat(),
    }
    return PrecisionPolicy(values, metadata, curves)


def manager_from_policy(policy: PrecisionPolicy, n_q: int, device, *, batch_size: int = 1,
                        capacity_tokens: int = 0, bit_v: int | None = None):
    """The packed cache for a policy: one tier table per layer, page and group sizes and the
    Value width from the metadata (defaults 128 / 128 / 128 / 2).  ``bit_v``, when given, must
    match the policy's (the reference adapter raises on a mismatch)."""
    from logitfill_amd.packed import PackedKVManager

    meta = policy.metadata
    saved_v = int(meta.get("bit_v", 2))
    if bit_v is not None and int(bit_v) != saved_v:
        raise ValueError(f"policy bit_v={saved_v} but the caller asks for bit_v={bit_v}")
    n_layers, n_kv, head_dim = policy.levels.shape
    if n_q % n_kv:
        raise ValueError(f"n_q {n_q} is not a multiple of the policy's {n_kv} kv heads")
    return PackedKVManager([policy.levels[layer] for layer in range(n_layers)], n_q, n_kv, head_dim,
                           int(meta.get("page_size", 128)), int(meta.get("k_group_size", 128)),
                           int(meta.get("v_group_size", 128)), saved_v, device, batch_size=batch_size,
                           capacity_tokens=capacity_tokens)
