"""The decode kernel's residual pass (the tail page and the new token) on both of its paths,
against the oracle (reference src/logitfill/packed/reference.py:30-56 over [history ; tail ;
new]): the matrix-core pass, taken for 2-byte tail and new-token rows of one dtype (bf16 or
fp16), and the VALU pass, taken for mixed dtypes and fp32 rows.  Tail lengths 0, 1, 63 and
127 (a full residual page), with and without a new token, alone (residual-only items) and
after packed pages (the residual shares an item with pages), at GQA 6 (two padding head
columns).  The oracle attends over the rows as stored: tail rows rounded to the tail's dtype,
the new token to its own."""
import numpy as np
import pytest
import torch

from logitfill_amd import _native, synth
from logitfill_amd.packed import PackedKVManager
from logitfill_amd.packed.reference import decode_into
from oracle import attention as oatt
from tests.helpers import assert_decode_close, f32

pytestmark = pytest.mark.gpu

B, N_Q, N_KV, D = 2, 12, 2, 128

DTYPES = [
    (torch.bfloat16, torch.bfloat16),   # matrix cores, bf16
    (torch.float16, torch.float16),     # matrix cores, fp16
    (torch.bfloat16, torch.float16),    # mixed: VALU
    (torch.float16, torch.float32),     # fp32 new token: VALU
    (torch.float32, torch.float32),     # fp32 rows: VALU
    (torch.float16, None),              # no new token: matrix cores, fp16
]


def _history(layer, b):
    hk, hv = layer.export_reference(b)
    if hk is None:
        return None, None
    return ({t: {k: v.cpu().numpy() for k, v in d.items()} for t, d in hk.items()},
            {k: v.cpu().numpy() for k, v in hv.items()})


@pytest.mark.parametrize("tail_dtype,new_dtype", DTYPES)
@pytest.mark.parametrize("pages,tail", [(0, 1), (0, 63), (2, 127), (3, 0)])
def test_residual_paths_match_oracle(gpu, tail_dtype, new_dtype, pages, tail):
    if tail == 0 and new_dtype is None and pages == 0:
        pytest.skip("nothing to attend")
    seed = 300 + 10 * pages + tail
    d = synth.make_layer(B, N_Q, N_KV, D, pages * 128 + 128, 2.5, seed=seed, device=gpu)
    mgr = PackedKVManager([d.levels], N_Q, N_KV, D, 128, 128, 128, 2, gpu, batch_size=B,
                          capacity_tokens=max(pages, 1) * 128)
    st = mgr.layers[0]
    if pages:
        st.fill_pages(d.key, d.value, [pages] * B)
    rk = d.key[:, :, pages * 128:pages * 128 + 127].to(tail_dtype)
    rv = d.value[:, :, pages * 128:pages * 128 + 127].to(tail_dtype)
    st.set_tail(rk, rv, [tail] * B)
    kn = None if new_dtype is None else d.key_new.to(new_dtype)
    vn = None if new_dtype is None else d.value_new.to(new_dtype)
    scaling = D ** -0.5
    out = torch.empty(B, N_Q, D, dtype=torch.float32, device=gpu)
    decode_into(mgr, 0, d.query, kn, vn, scaling, out, kernel=_native.KERNEL_MFMA)
    torch.cuda.synchronize()
    tk, tv = st.tail_buffers()
    for b in range(B):
        hk, hv = _history(st, b)
        store = oatt.ExportedHistory(d.levels, hk, hv, st.hist_lens[b], f32(tk[b, :, :tail]), f32(tv[b, :, :tail]),
                                     128, 128, 2)
        k_new = np.zeros((N_KV, 0, D), np.float32) if kn is None else f32(kn[b])[:, None, :]
        v_new = np.zeros((N_KV, 0, D), np.float32) if vn is None else f32(vn[b])[:, None, :]
        ref = oatt.reference_attention(store, f32(d.query[b])[:, None, :], k_new, v_new, scaling, N_Q, N_KV)[:, 0, :]
        print(f"residual: tail {tail_dtype} x {tail}, new {new_dtype}, pages {pages}, sequence {b}", flush=True)
        assert_decode_close(out[b], ref, out_dtype="fp32")


@pytest.mark.parametrize("kernel", [_native.KERNEL_MFMA, _native.KERNEL_VALU])
def test_full_tail_length_is_clamped_alike(gpu, kernel):
    """A raw caller that leaves tail_len at page_size (a full residual page not yet packed) gets
    the same result from both kernels: each clamps tail_len to min(tail_cap, page_size - 1), as
    the header documents, so the page's last row is left out -- the result equals a decode with
    tail_len 127, bit for bit, whatever that row holds."""
    d = synth.make_layer(B, N_Q, N_KV, D, 2 * 128 + 128, 2.5, seed=391, device=gpu)
    mgr = PackedKVManager([d.levels], N_Q, N_KV, D, 128, 128, 128, 2, gpu, batch_size=B, capacity_tokens=256)
    st = mgr.layers[0]
    st.fill_pages(d.key, d.value, [2] * B)
    st.set_tail(d.key[:, :, 256:383], d.value[:, :, 256:383], [127] * B)
    scaling = D ** -0.5
    want = torch.empty(B, N_Q, D, dtype=torch.float32, device=gpu)
    decode_into(mgr, 0, d.query, d.key_new, d.value_new, scaling, want, kernel=kernel)
    tk, tv = st.tail_buffers()
    tk[:, :, 127].copy_(d.key[:, :, 383] * 50)      # a row that would move the result
    tv[:, :, 127].copy_(d.value[:, :, 383] * 50)
    st.tail_len_device().fill_(128)                 # what a raw ABI caller might pass
    got = torch.empty_like(want)
    decode_into(mgr, 0, d.query, d.key_new, d.value_new, scaling, got, kernel=kernel)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
