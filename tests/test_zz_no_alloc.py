"""lf_decode_attention_noalloc (no counterpart in the reference; for callers that cannot
allocate): called through the C ABI, its output equals lf_decode_attention's bit for bit --
the same kernels, with the split-K partials in the library's per-GPU scratch array instead of
a caller workspace -- on consecutive calls (the second with a smaller input, so the array
still holds the first call's partials), for both decode kernels and multi-token queries; a
call whose partials exceed the array is refused before anything is enqueued."""
import ctypes

import pytest
import torch

from logitfill_amd import _native
from logitfill_amd.packed.reference import DecodePlan, decode_into, residual_pages
from tests.test_gpu_fullsize import _build

pytestmark = pytest.mark.gpu


def _pair(d, mgr, gpu, kernel, q_len=1):
    scaling = 128 ** -0.5
    if q_len == 1:
        q, kn, vn = d.query, d.key_new, d.value_new
    else:
        B, n_q, D = d.query.shape
        n_kv = d.key_new.shape[1]
        g = torch.Generator(device=gpu).manual_seed(q_len)
        q = (torch.randn(B, n_q, q_len, D, device=gpu, generator=g) * D ** -0.5).to(torch.bfloat16)
        kn = torch.randn(B, n_kv, q_len, D, device=gpu, generator=g).to(torch.bfloat16)
        vn = torch.randn(B, n_kv, q_len, D, device=gpu, generator=g).to(torch.bfloat16)
    ref = torch.empty_like(q)
    out = torch.full_like(q, float("nan"))
    decode_into(mgr, 0, q, kn, vn, scaling, ref, kernel=kernel)
    decode_into(mgr, 0, q, kn, vn, scaling, out, kernel=kernel, noalloc=True)
    torch.cuda.synchronize()
    return ref, out


@pytest.mark.parametrize("kernel", [_native.KERNEL_AUTO, _native.KERNEL_VALU])
def test_noalloc_equals_workspace_decode_on_consecutive_calls(gpu, kernel):
    d1, m1 = _build(gpu, 4, 28, 4, [40, 7, 33, 12], [50, 0, 127, 3], 2.5, seed=31)
    ref, out = _pair(d1, m1, gpu, kernel)
    assert torch.equal(ref, out)
    d2, m2 = _build(gpu, 2, 12, 2, [5, 2], [3, 90], 2.5, seed=32)   # smaller: fewer items, heads, rows
    ref2, out2 = _pair(d2, m2, gpu, kernel)
    assert torch.equal(ref2, out2)
    assert m2.layers[0].decode_plan.n_work < m1.layers[0].decode_plan.n_work


def test_noalloc_multi_token_queries(gpu):
    d, m = _build(gpu, 2, 8, 2, [6, 3], [20, 5], 3.0, seed=33)
    ref, out = _pair(d, m, gpu, _native.KERNEL_AUTO, q_len=3)
    assert torch.equal(ref, out)


def test_noalloc_refuses_partials_beyond_the_array(gpu):
    lib = _native.load()
    limit = lib.lf_noalloc_scratch_bytes()
    assert limit == 16 << 20
    d, m = _build(gpu, 1, 28, 4, [4], [2], 2.5, seed=34)
    layer = m.layers[0]
    n_work = limit // lib.lf_decode_workspace_bytes(28, 128, 1) + 1       # one item past the limit
    plan = DecodePlan([4], 4, 1, gpu, residual_pages([2]))
    a = _native.DecodeArgs()
    # query and out stay NULL: were the size check to regress, the call would fall through to
    # the argument checks and return LF_E_NULL without launching anything
    a.q_dtype, a.out_dtype = _native.LF_BF16, _native.LF_BF16
    a.tail_len = layer.tail_len_device().data_ptr()
    a.n_q, a.scaling, a.q_len = 28, 1.0, 1
    a.work, a.seq_work, a.n_work = plan.work.data_ptr(), plan.seq_work.data_ptr(), n_work
    st = lib.lf_decode_attention_noalloc(layer.layer_struct(), a, _native.current_stream_ptr(gpu))
    assert st == _native.LF_E_WORKSPACE
    assert b"workspace" in lib.lf_status_string(st)
