"""BF16 dense decode comparator (lf_dense_decode) against a float32 torch attention of the same
bf16 inputs.  Bar: max-abs 2e-3 (or one bf16 ulp) and rel-L2 1e-3 on the bf16 output."""
import numpy as np
import pytest
import torch

from helpers import assert_decode_close
from logitfill_amd.packed.dense import dense_decode

pytestmark = pytest.mark.gpu


def torch_reference(q, k, v, scaling, tokens):
    """float32 attention: softmax(q k^T * scaling) v over the first ``tokens`` positions, GQA by
    repeating each kv head over its g query heads (reference.py:10-15 repeat_kv)."""
    B, n_q, D = q.shape
    n_kv = k.shape[1]
    g = n_q // n_kv
    kf = k[:, :, :tokens].float().repeat_interleave(g, dim=1)   # [B, n_q, T, D]
    vf = v[:, :, :tokens].float().repeat_interleave(g, dim=1)
    s = torch.einsum("bhd,bhtd->bht", q.float(), kf) * scaling
    p = torch.softmax(s, dim=-1)
    return torch.einsum("bht,bhtd->bhd", p, vf)


def make(B, n_kv, g, T, seed, cap=None, scale_k=1.0):
    gen = torch.Generator().manual_seed(seed)
    cap = cap or T
    q = (torch.randn(B, n_kv * g, 128, generator=gen) / 128 ** 0.5).bfloat16()
    k = (torch.randn(B, n_kv, cap, 128, generator=gen) * scale_k).bfloat16()
    v = torch.randn(B, n_kv, cap, 128, generator=gen).bfloat16()
    return q, k, v


@pytest.mark.parametrize("B,n_kv,g,T,tps", [(1, 4, 7, 1024, 256), (2, 2, 7, 300, 128), (3, 1, 8, 1000, 384),
                                             (2, 3, 1, 129, 128), (1, 2, 5, 4096, 1024)])
def test_dense_decode_matches_fp32(gpu, B, n_kv, g, T, tps):
    q, k, v = make(B, n_kv, g, T, seed=B * 100 + T)
    out = dense_decode(q.to(gpu), k.to(gpu), v.to(gpu), 128 ** -0.5, tokens_per_split=tps)
    torch.cuda.synchronize()
    ref = torch_reference(q, k, v, 128 ** -0.5, T)
    assert_decode_close(out.cpu(), ref.numpy())


def test_dense_decode_strided_capacity_and_large_scores(gpu):
    """K/V as the first T rows of a larger capacity buffer; K scaled so scores span a wide range
    (exercises the lazy rescale)."""
    B, n_kv, g, T, cap = 2, 2, 7, 777, 1024
    q, k, v = make(B, n_kv, g, T, seed=7, cap=cap, scale_k=8.0)
    out = dense_decode(q.to(gpu), k.to(gpu), v.to(gpu), 128 ** -0.5, tokens=T, tokens_per_split=256)
    torch.cuda.synchronize()
    assert_decode_close(out.cpu(), torch_reference(q, k, v, 128 ** -0.5, T).numpy())


def test_dense_decode_split_invariance(gpu):
    q, k, v = make(1, 4, 7, 2048, seed=3)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    a = dense_decode(qd, kd, vd, 128 ** -0.5, tokens_per_split=128).float()
    b = dense_decode(qd, kd, vd, 128 ** -0.5, tokens_per_split=2048).float()
    torch.cuda.synchronize()
    assert float((a - b).abs().max()) <= 1e-2 * float(b.abs().max()) + 2e-3
