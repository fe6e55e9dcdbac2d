"""Host wiring of the model-integration caller (logitfill_amd/qwen2.py), on the CPU: with an
exact in-memory cache and dense attention standing in for the packed manager and kernel,
prefill + teacher-forced decode reproduce the unmodified model's full-sequence logits, which
pins the layer order (attention, then commit), the output transpose and the positions."""
import math

import torch

from logitfill_amd.qwen2 import PackedDecoder, detach_packed


class _ExactCache:
    def __init__(self, n_layers, n_kv, head_dim):
        self.layers = [None] * n_layers
        self.n_kv, self.head_dim = n_kv, head_dim
        self.k = [[] for _ in range(n_layers)]
        self.v = [[] for _ in range(n_layers)]

    def reset(self):
        for lst in self.k + self.v:
            lst.clear()

    def layer_length(self, layer):
        return sum(t.shape[2] for t in self.k[layer])

    def commit(self, layer, key, value):
        self.k[layer].append(key.detach().clone())
        self.v[layer].append(value.detach().clone())


def _exact_attention(cache, layer, query, key_new, value_new, scaling):
    k = torch.cat(cache.k[layer] + [key_new], dim=2)
    v = torch.cat(cache.v[layer] + [value_new], dim=2)
    g = query.shape[1] // k.shape[1]
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    s = torch.matmul(query, k.transpose(-1, -2).contiguous()) * scaling
    q_len, k_len = query.shape[2], k.shape[2]
    mask = torch.ones(q_len, k_len, dtype=torch.bool).tril(k_len - q_len)
    s = s.masked_fill(~mask, -math.inf)
    return torch.matmul(torch.softmax(s, dim=-1), v)


def test_decoder_wiring_reproduces_the_model():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      rope_theta=10000.0, attn_implementation="eager")
    torch.manual_seed(0)
    model = Qwen2ForCausalLM(cfg).float().eval()
    ids = torch.randint(0, 256, (1, 30), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = model(input_ids=ids, use_cache=False).logits[0]
    cache = _ExactCache(2, 2, 64)
    dec = PackedDecoder(model, cache, _exact_attention)
    got = [dec.prefill(ids[:, :20])]
    for t in range(20, 30):
        got.append(dec.step(ids[0, t]))
    detach_packed(model)
    got = torch.cat(got)
    assert torch.allclose(got, want[19:], atol=1e-4, rtol=1e-4)
    assert cache.layer_length(0) == 30 and cache.layer_length(1) == 30
    # three more positions at once (q_len 3): the output transpose keeps heads and positions apart
    dec = PackedDecoder(model, cache, _exact_attention)
    dec.prefill(ids[:, :27])
    with torch.no_grad():
        pos = torch.arange(27, 30).view(1, -1)
        multi = model(input_ids=ids[:, 27:], position_ids=pos, use_cache=False).logits[0]
    detach_packed(model)
    assert torch.allclose(multi, want[27:], atol=1e-4, rtol=1e-4)


class _ExactCacheWithLength(_ExactCache):
    """The exact cache plus the manager's ``seq_len`` (the last layer's length, as the
    reference manager updates it at the last layer's commit)."""

    @property
    def seq_len(self):
        return self.layer_length(len(self.layers) - 1)


def _small_model():
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=256, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      rope_theta=10000.0, attn_implementation="eager")
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).float().eval()


def test_logitfill_cache_shim_on_installed_transformers():
    """LogitFillCache (reference packed/cache.py:149-183) constructs on transformers 5.x and
    answers lengths and mask sizes from the manager; writes and beam search are refused."""
    from logitfill_amd.packed.cache import LogitFillCache

    cache = _ExactCacheWithLength(2, 2, 64)
    hf = LogitFillCache(cache)
    assert hf.get_seq_length() == 0 and hf.get_mask_sizes(5, 0) == (5, 0)
    cache.commit(0, torch.zeros(1, 2, 7, 64), torch.zeros(1, 2, 7, 64))
    cache.commit(1, torch.zeros(1, 2, 7, 64), torch.zeros(1, 2, 7, 64))
    assert hf.get_seq_length() == 7 and hf.get_query_offset() == 7
    assert hf.get_mask_sizes(1, 0) == (8, 0)
    assert hf.get_mask_sizes(torch.arange(3), 0) == (10, 0)  # transformers 4.x passes cache positions
    assert not hf.is_compileable and hf.get_max_length() == -1
    try:
        hf.update(None, None, 0)
        raise AssertionError("update must raise")
    except RuntimeError:
        pass
    try:
        hf.reorder_cache(torch.arange(1))
        raise AssertionError("reorder_cache must raise")
    except NotImplementedError:
        pass
    hf.reset()
    assert hf.get_seq_length() == 0


def test_generate_through_logitfill_cache_matches_plain_generate():
    """``model.generate(..., past_key_values=LogitFillCache(manager))`` -- the reference
    adapter's ``make_cache`` path (deepseek_qwen.py:141-146) -- decodes the same greedy tokens
    as the unmodified model without a cache, and PackedDecoder(hf_cache=True) gives the same
    logits as PackedDecoder with explicit positions."""
    from logitfill_amd.packed.cache import LogitFillCache
    from logitfill_amd.qwen2 import attach_packed

    model = _small_model()
    ids = torch.randint(0, 256, (1, 20), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        want = model.generate(ids, max_new_tokens=8, do_sample=False, use_cache=False)
    cache = _ExactCacheWithLength(2, 2, 64)
    attach_packed(model, cache, _exact_attention)
    with torch.no_grad():
        got = model.generate(ids, max_new_tokens=8, do_sample=False, past_key_values=LogitFillCache(cache),
                             use_cache=True)
    detach_packed(model)
    assert torch.equal(got, want)
    assert cache.layer_length(0) == 27  # prompt + 7 committed decode inputs

    runs = []
    for hf_cache in (False, True):
        dec = PackedDecoder(model, _ExactCacheWithLength(2, 2, 64), _exact_attention, hf_cache=hf_cache)
        steps = [dec.prefill(ids)]
        for t in range(5):
            steps.append(dec.step(want[0, 20 + t]))
        detach_packed(model)
        runs.append(torch.cat(steps))
    assert torch.allclose(runs[0], runs[1], atol=1e-5, rtol=1e-5)
