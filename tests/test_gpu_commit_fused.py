"""The commit folded into the decode launch (``packed_attention(..., commit=True)``,
``lf_decode_args.commit_new``) against the reference order -- ``packed_attention`` then
``manager.commit`` (reference ``qwen2_attention.py:223-256``, ``cache.py:135-140``): two managers
built from the same data decode the same tokens step by step across a residual page boundary;
every step's output is bit-identical and so are the layers' lengths, tail rows and packed
pages, for both decode kernels, for two new tokens per step and for a 32-head group on one kv
head (four row tiles per kv head, the first of which commits)."""
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import packed_attention

pytestmark = pytest.mark.gpu

D = 128


def _manager(gpu, d, B, n_q, n_kv, pages, tail):
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B,
                          capacity_tokens=(pages + 2) * 128)
    st = mgr.layers[0]
    st.fill_pages(d.key, d.value, [pages] * B)
    st.set_tail(d.key[:, :, pages * 128:pages * 128 + tail], d.value[:, :, pages * 128:pages * 128 + tail], [tail] * B)
    return mgr


def _same_state(a, b):
    la, lb = a.layers[0], b.layers[0]
    assert la.hist_lens == lb.hist_lens and la.tail_lens == lb.tail_lens and a.seq_len == b.seq_len
    assert torch.equal(la.tail_len_device(), lb.tail_len_device())
    assert la.tail_len_device().cpu().tolist() == la.tail_lens
    ta, tb = la.tail_buffers(), lb.tail_buffers()
    for x, y in zip(ta, tb):
        for s, n in enumerate(la.tail_lens):
            assert torch.equal(x[s, :, :n], y[s, :, :n])
    for s in range(la.batch):
        ha, va = la.export_reference(s)
        hb, vb = lb.export_reference(s)
        for t in range(4):
            for k in ha[t]:
                assert torch.equal(ha[t][k], hb[t][k]), (s, t, k)
        for k in va:
            assert torch.equal(va[k], vb[k]), (s, k)


@pytest.mark.parametrize("kernel,q_len,n_q,n_kv", [("auto", 1, 28, 4), ("valu", 1, 28, 4), ("auto", 2, 28, 4),
                                                  ("auto", 1, 32, 1)])
def test_folded_commit_matches_attention_then_commit(gpu, monkeypatch, kernel, q_len, n_q, n_kv):
    monkeypatch.setenv("LOGITFILL_AMD_KERNEL", kernel)
    B, pages, tail = 3, 6, 122
    d = synth.make_layer(B, n_q, n_kv, D, pages * 128 + 128, 2.5, seed=83, device=gpu)
    ref, fused = (_manager(gpu, d, B, n_q, n_kv, pages, tail) for _ in range(2))
    gen = torch.Generator(device=gpu).manual_seed(5)
    folded = 0
    for step in range(8):      # the tail reaches the page's end and a page is packed
        q = torch.randn(B, n_q, q_len, D, device=gpu, generator=gen).to(torch.bfloat16)
        k = torch.randn(B, n_kv, q_len, D, device=gpu, generator=gen).to(torch.bfloat16)
        v = torch.randn(B, n_kv, q_len, D, device=gpu, generator=gen).to(torch.bfloat16)
        before = fused.layers[0].tail_lens[0]
        out_r = packed_attention(ref, 0, q, k, v, D ** -0.5)
        ref.commit(0, k, v)
        out_f = packed_attention(fused, 0, q, k, v, D ** -0.5, commit=True)
        torch.cuda.synchronize()
        folded += int(before + q_len < 128)
        print(f"folded commit: kernel {kernel} q_len {q_len} heads {n_q}/{n_kv} step {step} tail {before}", flush=True)
        assert torch.equal(out_r, out_f)
        _same_state(ref, fused)
    assert ref.layers[0].hist_lens[0] == (pages + 1) * 128 and 0 < folded < 8
