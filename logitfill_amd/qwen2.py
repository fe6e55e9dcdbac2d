"""Qwen2 decoder on the packed backend: the model-integration caller of the decode path.

The reference patches every ``Qwen2Attention.forward`` so that, with the ``packed`` backend,
a layer with history runs ``packed_attention`` over the packed cache and every layer then
commits its new Key/Value states (attention first, then commit: completed pages are
compressed after the attention that produced them), while a layer with no history (the
prefill) runs the model's own dense attention (``src/logitfill/models/qwen2_attention.py:
76-146,223-256``; adapter ``models/deepseek_qwen.py:123-146``).

``attach_packed(model, manager)`` does the same for the installed transformers (5.x
``Qwen2Attention.forward(hidden_states, position_embeddings, attention_mask,
past_key_values=None, **kwargs)``), with two differences: the packed output
``[B, n_q, q_len, D]`` is transposed to the ``[B, q_len, n_q, D]`` the projection expects (the
reference reshapes it directly, which is right only for ``q_len == 1``), and the model runs
without a transformers cache -- the packed cache holds the history, so callers pass explicit
``position_ids`` (``PackedDecoder`` does).  ``detach_packed`` restores the original forwards.
"""
from __future__ import annotations

import torch

from logitfill_amd.packed.reference import packed_attention


def _dense_attention(attn, query, key, value, attention_mask, kwargs):
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    from transformers.models.qwen2.modeling_qwen2 import eager_attention_forward

    impl = ALL_ATTENTION_FUNCTIONS.get_interface(attn.config._attn_implementation, eager_attention_forward)
    out, _ = impl(attn, query, key, value, attention_mask, dropout=0.0, scaling=attn.scaling,
                  sliding_window=getattr(attn, "sliding_window", None), **kwargs)
    return out  # [B, q_len, n_q, D]


def _make_forward(attn, manager, attention_fn):
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    layer_idx = attn.layer_idx

    def forward(hidden_states, position_embeddings, attention_mask=None, past_key_values=None, **kwargs):
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, attn.head_dim)
        query = attn.q_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        key = attn.k_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        value = attn.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        query, key = apply_rotary_pos_emb(query, key, cos, sin)
        past = manager.layer_length(layer_idx)
        if past == 0:
            out = _dense_attention(attn, query, key, value, attention_mask, kwargs)
            manager.commit(layer_idx, key, value)
        elif attention_fn is packed_attention:
            # attention then commit, the commit folded into the decode launch where it can be
            out = packed_attention(manager, layer_idx, query, key, value, attn.scaling, commit=True).transpose(1, 2)
        else:
            out = attention_fn(manager, layer_idx, query, key, value, attn.scaling).transpose(1, 2)
            manager.commit(layer_idx, key, value)
        if past_key_values is not None and hasattr(past_key_values, "note_layer"):
            past_key_values.note_layer(layer_idx, manager.seq_len)  # LogitFillCache (qwen2_attention.py:254-255)
        out = out.reshape(*input_shape, -1).contiguous()
        return attn.o_proj(out), None

    return forward


def attach_packed(model, manager, attention_fn=packed_attention) -> None:
    """Route every decoder layer's attention through ``manager`` (a ``PackedKVManager`` whose
    layers match the model's).  ``attention_fn`` is ``packed_attention`` (the HIP path) or
    ``reference_attention`` (dense dequantise-then-attend), same signature."""
    cfg = model.config
    n_kv = int(cfg.num_key_value_heads)
    layers = model.model.layers
    if len(manager.layers) != len(layers):
        raise ValueError(f"manager has {len(manager.layers)} layers, the model {len(layers)}")
    for layer in layers:
        attn = layer.self_attn
        if manager.n_kv != n_kv or manager.head_dim != attn.head_dim:
            raise ValueError("manager shape does not match the model's attention")
        if not hasattr(attn, "_lf_original_forward"):
            attn._lf_original_forward = attn.forward
        attn.forward = _make_forward(attn, manager, attention_fn)


def detach_packed(model) -> None:
    for layer in model.model.layers:
        attn = layer.self_attn
        if hasattr(attn, "_lf_original_forward"):
            attn.forward = attn._lf_original_forward
            del attn._lf_original_forward


class PackedDecoder:
    """Prefill + token-by-token decode of a ``Qwen2ForCausalLM`` over a packed cache (batch 1,
    as the reference).  ``step`` returns the logits of the last position.

    ``hf_cache=True`` passes a ``LogitFillCache`` as ``past_key_values`` (the reference adapter's
    ``make_cache``, ``deepseek_qwen.py:141-146``), so the model derives positions and mask sizes
    from the packed length; otherwise the decoder passes the positions itself.

    ``defer_flush``: None (default) keeps the manager's own setting; True or False sets it on
    the manager.  A deferring manager leaves every layer's completed page for one
    ``flush_pending`` launch after each forward pass (``step`` calls it) instead of one launch
    per layer; results are the same either way."""

    def __init__(self, model, manager, attention_fn=packed_attention, *, hf_cache: bool = False,
                 defer_flush: bool | None = None):
        self.model, self.manager = model, manager
        if defer_flush is not None and hasattr(manager, "defer_flush"):
            manager.defer_flush = bool(defer_flush)
        attach_packed(model, manager, attention_fn)
        self.cache = None
        if hf_cache:
            from logitfill_amd.packed.cache import LogitFillCache

            self.cache = LogitFillCache(manager)
        self.pos = 0

    def _flush(self) -> None:
        flush = getattr(self.manager, "flush_pending", None)  # managers without deferral have none
        if flush is not None:
            flush()

    def _forward(self, ids: torch.Tensor, start: int) -> torch.Tensor:
        if self.cache is not None:
            out = self.model(input_ids=ids, past_key_values=self.cache, use_cache=True)
        else:
            pos = torch.arange(start, start + ids.shape[-1], device=ids.device)[None]
            out = self.model(input_ids=ids, position_ids=pos, use_cache=False)
        self._flush()
        return out.logits[:, -1]

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        self.manager.reset()
        logits = self._forward(input_ids, 0)
        self.pos = int(input_ids.shape[-1])
        return logits

    @torch.no_grad()
    def step(self, token: torch.Tensor) -> torch.Tensor:
        logits = self._forward(token.view(1, 1), self.pos)
        self.pos += 1
        return logits
