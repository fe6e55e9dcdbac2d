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


def test_packed_decoder_layers_match_the_oracle(gpu):
    """Row f1 against the oracle: every packed attention call of a decode across a page flush
    (each layer, each step) meets the north-star bar against the oracle's dense path over that
    layer's exported history, and at the end every layer's packed history equals the oracle's
    pack of all the Keys and Values the model committed to it (bit for bit)."""
    from oracle import attention as oatt
    from tests.helpers import assert_decode_close, assert_history_equal, oracle_store

    model = _model(gpu)
    mgr = _manager(gpu)
    committed = {0: [], 1: []}
    commit = mgr.commit

    def recording_commit(layer_idx, key, value, lengths=None):
        committed[layer_idx].append((key.detach().float().cpu(), value.detach().float().cpu()))
        commit(layer_idx, key, value, lengths)

    mgr.commit = recording_commit
    checked = []

    def checked_attention(manager, layer_idx, query, key_new, value_new, scaling):
        out = packed_attention(manager, layer_idx, query, key_new, value_new, scaling)
        st = manager.layers[layer_idx]
        hk, hv = st.export_reference(0)
        hk = {t: {k: v.cpu().numpy() for k, v in d.items()} for t, d in hk.items()}
        hv = {k: v.cpu().numpy() for k, v in hv.items()}
        tl = st.tail_lens[0]
        tk, tv = st.tail_buffers()
        tail_k = tk[0, :, :tl].float().cpu().numpy() if tl else None
        tail_v = tv[0, :, :tl].float().cpu().numpy() if tl else None
        store = oatt.ExportedHistory(levels[layer_idx], hk, hv, st.hist_lens[0], tail_k, tail_v, 128, 128, 2)
        ref = oatt.reference_attention(store, query[0].float().cpu().numpy(), key_new[0].float().cpu().numpy(),
                                       value_new[0].float().cpu().numpy(), scaling, 4, 2)
        assert_decode_close(out[0], ref, out_dtype="fp32")
        checked.append(layer_idx)
        return out

    levels = [synth.sample_tier_levels(2, 128, 2.5, seed=s) for s in range(2)]
    g = torch.Generator().manual_seed(7)
    prompt = torch.randint(0, 512, (1, 250), generator=g).to(gpu)
    forced = torch.randint(0, 512, (12,), generator=g).to(gpu)   # page flush at position 256
    dec = PackedDecoder(model, mgr, checked_attention)
    dec.prefill(prompt)
    for tok in forced:
        dec.step(tok)
    detach_packed(model)
    assert len(checked) == 2 * len(forced)
    for layer in range(2):
        keys = torch.cat([k for k, _ in committed[layer]], dim=2)[0].numpy()
        values = torch.cat([v for _, v in committed[layer]], dim=2)[0].numpy()
        assert keys.shape[1] == 250 + 12
        assert_history_equal(mgr.layers[layer], 0, oracle_store(levels[layer], keys, values))


def test_generate_with_logitfill_cache_on_the_packed_backend(gpu):
    """``model.generate(..., past_key_values=LogitFillCache(manager))`` on the HIP path (the
    reference adapter's make_cache, deepseek_qwen.py:141-146) produces the same greedy tokens
    as PackedDecoder stepping the same manager shape with explicit positions."""
    from logitfill_amd.packed.cache import LogitFillCache
    from logitfill_amd.qwen2 import attach_packed

    model = _model(gpu)
    g = torch.Generator().manual_seed(9)
    prompt = torch.randint(0, 512, (1, 120), generator=g).to(gpu)
    mgr = _manager(gpu)
    attach_packed(model, mgr)
    with torch.no_grad():
        gen = model.generate(prompt, max_new_tokens=12, do_sample=False, past_key_values=LogitFillCache(mgr),
                             use_cache=True)
    detach_packed(model)
    assert mgr.seq_len == 120 + 11 and mgr.layers[0].hist_len == 128
    dec = PackedDecoder(model, _manager(gpu))
    logits = dec.prefill(prompt)
    tokens = []
    for _ in range(12):
        tok = int(logits.argmax(-1))
        tokens.append(tok)
        logits = dec.step(torch.tensor(tok, device=gpu))
    detach_packed(model)
    assert gen[0, 120:].tolist() == tokens
