"""Model-integration caller (reference src/logitfill/models/qwen2_attention.py:76-146,223-256):
a small random-weight Qwen2ForCausalLM decodes on the packed backend; its logits match the
same model driven through the dense dequantise-then-attend path over an identically filled
packed cache, step by step across a page flush.  float32 model (no bf16 batched products)."""
import numpy as np
import pytest
import torch

from logitfill_amd import synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import packed_attention, reference_attention
from logitfill_amd.qwen2 import PackedDecoder, detach_packed

pytestmark = pytest.mark.gpu


def _model(dev):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=2048,
                      rope_theta=10000.0, attn_implementation="eager")
    torch.manual_seed(0)
    return Qwen2ForCausalLM(cfg).to(dev).float().eval()


def _manager(dev, defer_flush=False):
    levels = [synth.sample_tier_levels(2, 128, 2.5, seed=s) for s in range(2)]
    return PackedKVManager(levels, 4, 2, 128, 128, 128, 128, 2, dev, defer_flush=defer_flush)


def _run(model, dev, attention_fn, prompt, forced, defer_flush=False):
    mgr = _manager(dev, defer_flush)
    dec = PackedDecoder(model, mgr, attention_fn)
    out = [dec.prefill(prompt).float()]
    for tok in forced:
        out.append(dec.step(tok).float())
    detach_packed(model)
    return torch.cat(out), mgr


def test_packed_decoder_matches_dense_dequant_path(gpu):
    model = _model(gpu)
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 512, (1, 370), generator=g).to(gpu)
    forced = torch.randint(0, 512, (20,), generator=g).to(gpu)  # page flush at position 384
    ours, mgr = _run(model, gpu, packed_attention, prompt, forced)
    ref, _ = _run(model, gpu, reference_attention, prompt, forced)
    assert mgr.layers[0].hist_len == 384 and mgr.layers[1].tail_len == 370 + 20 - 384
    for s in range(ours.shape[0]):
        rel = float((ours[s] - ref[s]).norm() / ref[s].norm())
        assert rel < 1e-3, f"step {s}: rel-L2 {rel:.3g}"
    # sanity against the unquantised model: the int2 Values of the random-weight model move the
    # logits (cosine 0.93-0.98 per step for this seed; unrelated logits would be near 0)
    with torch.no_grad():
        full = torch.cat([prompt[0], forced]).view(1, -1)
        dense = model(input_ids=full, use_cache=False).logits[0, 369:].float()
    cos = torch.nn.functional.cosine_similarity(ours, dense, dim=-1)
    assert float(cos[0]) > 0.999 and float(cos.min()) > 0.9, cos  # step 0: prefill, no quantised reads


def test_detach_restores_the_model(gpu):
    model = _model(gpu)
    ids = torch.arange(40, device=gpu).view(1, -1)
    with torch.no_grad():
        before = model(input_ids=ids, use_cache=False).logits
    dec = PackedDecoder(model, _manager(gpu))
    dec.prefill(ids)
    detach_packed(model)
    with torch.no_grad():
        after = model(input_ids=ids, use_cache=False).logits
    assert torch.equal(before, after)


def test_deferred_flushes_give_the_same_logits(gpu):
    """The decoder with deferred page flushes (both layers' page at position 384 packed by one
    lf_pack_pages_multi launch after the step) reproduces the eager-flush logits exactly."""
    model = _model(gpu)
    g = torch.Generator().manual_seed(5)
    prompt = torch.randint(0, 512, (1, 380), generator=g).to(gpu)
    forced = torch.randint(0, 512, (10,), generator=g).to(gpu)
    eager, _ = _run(model, gpu, packed_attention, prompt, forced)
    lazy, mgr = _run(model, gpu, packed_attention, prompt, forced, defer_flush=True)
    assert mgr.defer_flush and all(layer.pending == [] for layer in mgr.layers)
    assert mgr.layers[0].hist_len == 384 and mgr.layers[1].hist_len == 384
    assert torch.equal(eager, lazy)
