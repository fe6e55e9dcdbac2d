"""Tier-table policy files: the ``[n_layers, n_kv, head_dim]`` Key level map on disk.

Levels are 0 = int2, 1 = int4, 2 = int8, 3 = fp16.  The on-disk format is the
reference's (``src/logitfill/allocators/policy.py:68-86``), so calibrated tables
move between the two implementations unchanged:

* ``policy.npz`` -- array ``levels`` (int64, the level map) and one array per
  optional per-channel curve, each of the level map's shape;
* ``metadata.json`` -- a flat JSON object (sorted keys, two-space indent) whose
  keys are listed in ``METADATA_KEYS``.

Checks applied on construction and load: the level map is 3-D with values in
0..3; ``n_layers`` / ``n_kv`` / ``head_dim`` in the metadata agree with it;
every curve has its shape; and, when the metadata names a ``target_bit`` and
does not set ``enforce_budget`` to false, no kv head spends more Key bits above
the int2 floor than the budget allows (``src/logitfill/allocators/allocate.py:
14-88``): with the Value width ``bit_v`` fixed, a history target of
``target_bit`` bits per K/V element leaves ``2 * target_bit - bit_v`` bits per
Key element, i.e. ``round((2 * target_bit - bit_v - 2) * head_dim)`` bits per
head above int2, where an int4 / int8 / fp16 channel costs 2 / 6 / 14 of them.

``manager_from_policy`` builds the packed cache that consumes a policy (the
reference adapter's ``load_policy`` + ``packed_manager``,
``src/logitfill/models/deepseek_qwen.py:111-137``).  Archives are read with
``allow_pickle=False``.
"""
from __future__ import annotations

import json
from dataclasses import dataclass
from datetime import datetime, timezone
from pathlib import Path

import numpy as np

from logitfill_amd import __version__

POLICY_VERSION = 1
LEVEL_NAMES = ("int2", "int4", "int8", "fp16")
LEVEL_BITS = np.array([2, 4, 8, 16], dtype=np.int64)
# Key bits of one channel above the int2 floor, per level.
LEVEL_EXTRA = LEVEL_BITS - LEVEL_BITS[0]

# metadata.json keys written by build_policy (the reference's format).
METADATA_KEYS = (
    "policy_version", "code_version", "model_id", "n_layers", "n_kv", "head_dim", "k_group_size",
    "v_group_size", "page_size", "bit_v", "target_bit", "target_bit_k", "extra_budget_per_head",
    "calibration_datasets", "n_samples", "normalized", "histogram", "achieved", "created_utc",
)
_SHAPE_KEYS = ("n_layers", "n_kv", "head_dim")


def _level_map(levels, ndim: int | None = None) -> np.ndarray:
    arr = np.asarray(levels, dtype=np.int64)
    if ndim is not None and arr.ndim != ndim:
        raise ValueError(f"a level map must be [layers, kv_heads, head_dim]; got shape {arr.shape}")
    if arr.size and (arr.min() < 0 or arr.max() > 3):
        raise ValueError("level codes must lie in 0..3 (int2, int4, int8, fp16)")
    return arr


@dataclass(frozen=True)
class KeyBudget:
    """The per-head Key bit budget implied by a K/V history target."""

    target_bit: float
    bit_v: int = 2
    channels: int = 128

    def __post_init__(self):
        if not 2 <= int(self.bit_v) <= 16:
            raise ValueError(f"bit_v={self.bit_v}: the Value width must lie in 2..16 bits")
        if not 2.0 <= self.target_bit_k <= 16.0:
            raise ValueError(f"target_bit={self.target_bit} with bit_v={self.bit_v} asks for "
                             f"{self.target_bit_k} Key bits per element; the tiers span 2..16")

    @property
    def target_bit_k(self) -> float:
        """Key bits per element: the history average fixes K + V = 2 * target_bit."""
        return 2.0 * float(self.target_bit) - float(self.bit_v)

    @property
    def extra_bits(self) -> int:
        """Key bits one head may spend above the all-int2 floor."""
        return int(round((self.target_bit_k - 2.0) * self.channels))

    def as_dict(self) -> dict:
        return {"target_bit": float(self.target_bit), "bit_v": int(self.bit_v),
                "target_bit_k": float(self.target_bit_k), "extra_budget_per_head": self.extra_bits,
                "n_channels": int(self.channels)}


def extra_budget_per_head(target_bit_k: float, n_channels: int = 128) -> int:
    """Key bits per head above int2 for a Key target of ``target_bit_k`` bits per element."""
    extra = (float(target_bit_k) - 2.0) * n_channels
    if extra < 0:
        raise ValueError(f"a Key target of {target_bit_k} bits is below the 2-bit floor")
    return int(round(extra))


def kv_history_budget(target_bit: float, bit_v: int = 2, n_channels: int = 128) -> dict:
    """``KeyBudget(...).as_dict()``: the Key target and per-head extra bits of a K/V target."""
    return KeyBudget(float(target_bit), int(bit_v), int(n_channels)).as_dict()


def spent_extra_per_head(levels) -> np.ndarray:
    """Key bits above int2 that each head of a ``[..., head_dim]`` level map spends."""
    return LEVEL_EXTRA[_level_map(levels)].sum(axis=-1)


def achieved_history_bits(levels, bit_v: int = 2) -> dict:
    """Mean Key bits of a level map, the Value width, and their mean (the K/V history rate)."""
    arr = _level_map(levels)
    bit_k = float(LEVEL_BITS[arr].mean()) if arr.size else float("nan")
    return {"actual_bit_k": bit_k, "bit_v": float(bit_v), "actual_bit_kv": (bit_k + float(bit_v)) / 2.0}


def assert_history_budget(levels, target_bit: float, bit_v: int = 2) -> dict:
    """Check every head against its budget; returns the budget, the largest spend and the
    achieved rates, or raises ValueError naming the first head over budget."""
    arr = _level_map(levels)
    budget = KeyBudget(float(target_bit), int(bit_v), int(arr.shape[-1]))
    spent = spent_extra_per_head(arr)
    over = np.argwhere(spent > budget.extra_bits)
    if over.size:
        head = tuple(int(i) for i in over[0])
        raise ValueError(f"kv head {head} spends {int(spent[head])} Key bits above int2; "
                         f"target_bit={target_bit} allows {budget.extra_bits}")
    out = budget.as_dict()
    out["extra_spent_per_head"] = int(spent.max()) if spent.size else 0
    out.update(achieved_history_bits(arr, bit_v))
    return out


def level_histogram(levels) -> dict:
    """Mean number of channels per head at each level, and the mean Key bits."""
    arr = _level_map(levels)
    heads = max(1, arr.size // max(1, arr.shape[-1])) if arr.ndim else 1
    counts = np.bincount(arr.reshape(-1), minlength=4)
    hist = {name: float(counts[code]) / heads for code, name in enumerate(LEVEL_NAMES)}
    hist["actual_bit_k"] = float(LEVEL_BITS[arr].mean()) if arr.size else float("nan")
    return hist


def _model_basename(model_id) -> str:
    return str(model_id).replace("\\", "/").rstrip("/").rsplit("/", 1)[-1]


class PrecisionPolicy:
    """A checked Key level map ``levels [n_layers, n_kv, head_dim]`` with its metadata and
    optional per-channel ``curves`` (same shape as the levels)."""

    def __init__(self, levels, metadata: dict, curves: dict | None = None):
        self.levels = _level_map(levels, ndim=3)
        self.metadata = dict(metadata)
        self.curves = {str(name): np.asarray(arr) for name, arr in (curves or {}).items()}
        self.check()

    @property
    def shape(self) -> tuple[int, int, int]:
        return tuple(int(x) for x in self.levels.shape)

    def check(self) -> None:
        """Metadata/shape agreement, curve shapes and (unless disabled) the Key budget."""
        for axis, key in enumerate(_SHAPE_KEYS):
            if key in self.metadata and int(self.metadata[key]) != self.shape[axis]:
                raise ValueError(f"metadata says {key}={self.metadata[key]}, the level map is {self.shape}")
        bad = [name for name, arr in self.curves.items() if arr.shape != self.levels.shape]
        if bad:
            raise ValueError(f"curves {bad} do not have the level map's shape {self.shape}")
        if "target_bit" in self.metadata and self.metadata.get("enforce_budget", True):
            assert_history_budget(self.levels, float(self.metadata["target_bit"]),
                                  int(self.metadata.get("bit_v", 2)))

    def validate_model(self, model) -> None:
        """Raise ValueError unless ``model`` (or a model config) has this policy's
        ``(num_hidden_layers, num_key_value_heads, head_dim)`` and, where both sides name one,
        the same model (compared by the last path component of the id)."""
        cfg = getattr(model, "config", model)
        n_heads = int(cfg.num_attention_heads)
        head_dim = getattr(cfg, "head_dim", None) or int(cfg.hidden_size) // n_heads
        want = (int(cfg.num_hidden_layers), int(cfg.num_key_value_heads), int(head_dim))
        if self.shape != want:
            raise ValueError(f"the policy is {self.shape} (layers, kv heads, head dim); the model is {want}")
        mine = self.metadata.get("model_id")
        theirs = getattr(cfg, "name_or_path", None) or getattr(cfg, "_name_or_path", None)
        if mine and theirs and str(mine) != str(theirs) and _model_basename(mine) != _model_basename(theirs):
            raise ValueError(f"the policy was calibrated for {mine!r}, not {theirs!r}")

    def save(self, directory) -> Path:
        out = Path(directory)
        out.mkdir(parents=True, exist_ok=True)
        arrays = dict(self.curves)
        arrays["levels"] = self.levels
        np.savez_compressed(out / "policy.npz", **arrays)
        text = json.dumps(self.metadata, indent=2, sort_keys=True)
        (out / "metadata.json").write_text(text + "\n", encoding="utf-8")
        return out

    @classmethod
    def load(cls, directory) -> "PrecisionPolicy":
        src = Path(directory)
        with np.load(src / "policy.npz", allow_pickle=False) as npz:
            arrays = {name: np.array(npz[name]) for name in npz.files}
        if "levels" not in arrays:
            raise ValueError(f"{src / 'policy.npz'} holds no 'levels' array")
        metadata = json.loads((src / "metadata.json").read_text(encoding="utf-8"))
        return cls(arrays.pop("levels"), metadata, arrays)


def build_policy(levels, *, model_id: str, target_bit: float, bit_v: int = 2, k_group_size: int = 128,
                 v_group_size: int = 128, page_size: int = 128, calibration_datasets=None, n_samples: int = 0,
                 curves: dict | None = None, normalized: bool = True) -> PrecisionPolicy:
    """Wrap an allocator's level map as a checked policy with the metadata of ``METADATA_KEYS``."""
    arr = _level_map(levels, ndim=3)
    budget = assert_history_budget(arr, target_bit, bit_v)
    fields = {
        "policy_version": POLICY_VERSION,
        "code_version": __version__,
        "model_id": model_id,
        **dict(zip(_SHAPE_KEYS, (int(x) for x in arr.shape))),
        "k_group_size": int(k_group_size),
        "v_group_size": int(v_group_size),
        "page_size": int(page_size),
        "bit_v": int(bit_v),
        "target_bit": float(target_bit),
        "target_bit_k": budget["target_bit_k"],
        "extra_budget_per_head": budget["extra_budget_per_head"],
        "calibration_datasets": [str(x) for x in (calibration_datasets or [])],
        "n_samples": int(n_samples),
        "normalized": bool(normalized),
        "histogram": level_histogram(arr),
        "achieved": achieved_history_bits(arr, bit_v),
        "created_utc": datetime.now(timezone.utc).isoformat(),
    }
    metadata = {key: fields[key] for key in METADATA_KEYS}
    return PrecisionPolicy(arr, metadata, curves)


def manager_from_policy(policy: PrecisionPolicy, n_q: int, device, *, batch_size: int = 1,
                        capacity_tokens: int = 0, bit_v: int | None = None, defer_flush: bool = True):
    """The packed cache for ``policy``: one tier table per layer; page size, Key / Value groups
    and Value width from the metadata (defaults 128, 128, 128, 2).  A caller's ``bit_v`` must
    equal the policy's.  Page flushes are deferred to ``flush_pending`` by default (one launch
    per decode step for all layers)."""
    from logitfill_amd.packed import PackedKVManager

    meta = policy.metadata
    stored_v = int(meta.get("bit_v", 2))
    if bit_v is not None and int(bit_v) != stored_v:
        raise ValueError(f"the policy stores Values at {stored_v} bits; bit_v={bit_v} was asked for")
    n_layers, n_kv, head_dim = policy.shape
    if int(n_q) % n_kv:
        raise ValueError(f"{n_q} query heads do not split evenly over the policy's {n_kv} kv heads")
    return PackedKVManager(list(policy.levels), int(n_q), n_kv, head_dim, int(meta.get("page_size", 128)),
                           int(meta.get("k_group_size", 128)), int(meta.get("v_group_size", 128)), stored_v,
                           device, batch_size=batch_size, capacity_tokens=capacity_tokens,
                           defer_flush=defer_flush)
