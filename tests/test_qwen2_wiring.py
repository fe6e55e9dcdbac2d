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
