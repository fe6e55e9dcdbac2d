"""Query rows beyond one workgroup, on the decode kernels: several new tokens per sequence
(speculative decoding and chunked scoring, reference src/logitfill/packed/reference.py:18-27,48
-- query token j sees the history, the tail and new tokens 0..j), GQA groups wider than a
workgroup's row tile (MQA), new tokens that carry the residual past one 128-token chunk, and
head_dim 1024 (the largest head the reference kernel takes, kernel.cu:224-230).  Every case runs
on a packed-decode kernel -- ``packed_attention`` takes no dense fallback -- and meets the
north-star bar against the oracle's dense dequantise-then-attend path (reference.py:30-56)."""
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import DENSE_FALLBACKS, decode_into, packed_attention
from oracle import attention as oatt
from tests.helpers import assert_decode_close, f32, oracle_store

pytestmark = pytest.mark.gpu


def _case(gpu, n_q, n_kv, D, pages, tails, q_len, seed):
    """Manager with sequence b = pages[b] packed pages + tails[b] residual tokens, the q_len new
    tokens that follow them, and the oracle's float32 output per sequence ``[n_q, q_len, D]``."""
    B = len(pages)
    lens = [p * 128 + t for p, t in zip(pages, tails)]
    d = synth.make_layer(B, n_q, n_kv, D, max(lens) + q_len, 2.5, seed=seed)
    mgr = PackedKVManager([d.levels], n_q, n_kv, D, 128, 128, 128, 2, gpu, batch_size=B)
    mgr.commit(0, d.key[:, :, :max(lens)].to(gpu), d.value[:, :, :max(lens)].to(gpu), lengths=lens)
    q = (torch.randn(B, n_q, q_len, D, generator=torch.Generator().manual_seed(seed)) * D ** -0.5).bfloat16()
    kn = torch.stack([d.key[b, :, lens[b]:lens[b] + q_len] for b in range(B)])
    vn = torch.stack([d.value[b, :, lens[b]:lens[b] + q_len] for b in range(B)])
    refs = []
    for b in range(B):
        store = oracle_store(d.levels, f32(d.key[b, :, :lens[b]]), f32(d.value[b, :, :lens[b]]))
        refs.append(oatt.reference_attention(store, f32(q[b]), f32(kn[b]), f32(vn[b]), D ** -0.5, n_q, n_kv))
    return mgr, q.to(gpu), kn.to(gpu).contiguous(), vn.to(gpu).contiguous(), refs


def _check(out, refs, out_dtype="bf16"):
    for b, ref in enumerate(refs):
        for j in range(ref.shape[1]):
            assert_decode_close(out[b, :, j], ref[:, j], out_dtype=out_dtype)


def _decode(mgr, q, kn, vn, kernel, pages_per_split=None):
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    decode_into(mgr, 0, q, kn, vn, q.shape[-1] ** -0.5, out, kernel=kernel, pages_per_split=pages_per_split)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("q_len", [2, 4, 8])
def test_speculative_tokens_on_matrix_cores(gpu, q_len):
    """The 7B shape's GQA 7 (28 q / 4 kv heads) with 2, 4 and 8 new tokens: 14-56 rows per kv
    head, 2-7 row tiles of the matrix-core kernel; tails of 100 (c2's), 127 (with the new tokens
    the residual crosses a 128-token chunk), 0 and 40, one sequence with no packed page.  The
    automatic path (``packed_attention``) takes the matrix-core kernel and no dense fallback;
    the explicit kernel with split items meets the bar as well."""
    mgr, q, kn, vn, refs = _case(gpu, 28, 4, 128, [5, 3, 2, 0], [100, 127, 0, 40], q_len, seed=500 + q_len)
    before = dict(DENSE_FALLBACKS)
    out = packed_attention(mgr, 0, q, kn, vn, 128 ** -0.5)
    torch.cuda.synchronize()
    assert dict(DENSE_FALLBACKS) == before
    _check(out, refs)
    for pps in (None, 2):
        _check(_decode(mgr, q, kn, vn, _native.KERNEL_MFMA, pps), refs, "fp32")


@pytest.mark.parametrize("kernel", [_native.KERNEL_MFMA, _native.KERNEL_VALU])
def test_chunked_scoring_residual_past_one_chunk(gpu, kernel):
    """40 new tokens after tails of 100 and 127 tokens: the residual (tail + new tokens, 140 and
    167) spans two 128-token chunks, the causal mask reaches into the second, and 7 x 40 = 280
    rows per kv head make 35 matrix-core row tiles (18 VALU tiles)."""
    mgr, q, kn, vn, refs = _case(gpu, 28, 4, 128, [3, 1], [100, 127], 40, seed=540)
    _check(_decode(mgr, q, kn, vn, kernel), refs, "fp32")
    _check(_decode(mgr, q, kn, vn, kernel, pages_per_split=1), refs, "fp32")


@pytest.mark.parametrize("kernel", [_native.KERNEL_AUTO, _native.KERNEL_VALU])
@pytest.mark.parametrize("n_q,n_kv,q_len", [(32, 1, 1), (64, 2, 2), (24, 1, 1)])
def test_wide_query_groups(gpu, kernel, n_q, n_kv, q_len):
    """MQA and wide GQA groups, which the reference kernel serves (one block per q head,
    kernel.cu:234): 32 q heads on 1 kv head, 64 q on 2 with 2 new tokens (64 rows per kv head),
    and GQA 24; the automatic path takes the matrix-core kernel's row tiles."""
    mgr, q, kn, vn, refs = _case(gpu, n_q, n_kv, 128, [4, 9], [17, 120], q_len, seed=560 + n_q + q_len)
    if kernel == _native.KERNEL_AUTO:
        before = dict(DENSE_FALLBACKS)
        out = packed_attention(mgr, 0, q, kn, vn, 128 ** -0.5)
        torch.cuda.synchronize()
        assert dict(DENSE_FALLBACKS) == before
        _check(out, refs)
    _check(_decode(mgr, q, kn, vn, kernel, pages_per_split=3), refs, "fp32")


@pytest.mark.parametrize("q_len", [1, 3])
def test_head_dim_1024(gpu, q_len):
    """head_dim 1024 (pages packed by the general packer, decoded by the general kernel in tiles
    of 8 query rows): one and three new tokens, GQA 2, tails of 20 and 127."""
    mgr, q, kn, vn, refs = _case(gpu, 4, 2, 1024, [3, 1], [20, 127], q_len, seed=580 + q_len)
    before = dict(DENSE_FALLBACKS)
    out = packed_attention(mgr, 0, q, kn, vn, 1024 ** -0.5)
    torch.cuda.synchronize()
    assert dict(DENSE_FALLBACKS) == before
    _check(out, refs)
    _check(_decode(mgr, q, kn, vn, _native.KERNEL_AUTO, pages_per_split=1), refs, "fp32")
