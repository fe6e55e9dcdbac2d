"""Packed Key/Value history and its decode path on MI355X (reference ``logitfill.packed``)."""

from logitfill_amd.packed.cache import LogitFillCache, PackedKVManager

__all__ = ["LogitFillCache", "PackedKVManager"]
