"""ctypes binding of ``liblogitfill_amd.so`` (C ABI in ``include/logitfill_amd.h``).

The library is loaded lazily and only after ``torch`` is imported, so that its
``libamdhip64.so.7`` dependency binds to the HIP runtime torch already loaded
(one runtime, one set of streams per process).  A missing library raises
``NativeLibraryMissing``; there is no fallback.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int32, c_int64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("liblogitfill_amd.so")

LF_BF16, LF_FP16, LF_FP32 = 0, 1, 2
LF_OK, LF_E_NULL, LF_E_SHAPE, LF_E_UNSUPPORTED, LF_E_WORKSPACE, LF_E_DTYPE = 0, -1, -2, -3, -4, -5
KERNEL_AUTO, KERNEL_VALU, KERNEL_MFMA = 0, 1, 2


class NativeLibraryMissing(RuntimeError):
    """The HIP extension is not built; run ``python -m logitfill_amd.build``."""


class LFError(RuntimeError):
    """A C-ABI call returned a non-zero status."""

    def __init__(self, status: int, message: str, call: str):
        super().__init__(f"{call} failed with status {status}: {message}")
        self.status = status


class PackedLayer(ctypes.Structure):
    """``lf_packed_layer``."""

    _fields_ = [
        ("k_code", c_void_p * 3),
        ("k_scale", c_void_p * 3),
        ("k_min", c_void_p * 3),
        ("k_value16", c_void_p),
        ("v_code", c_void_p),
        ("v_scale", c_void_p),
        ("v_min", c_void_p),
        ("v_value16", c_void_p),
        ("tier_index", c_void_p * 4),
        ("tier_count", c_void_p * 4),
        ("batch", c_int32),
        ("n_kv", c_int32),
        ("head_dim", c_int32),
        ("cap_tokens", c_int32),
        ("cap_kgroups", c_int32),
        ("page_size", c_int32),
        ("k_group", c_int32),
        ("v_group", c_int32),
        ("bit_v", c_int32),
        ("k_width", c_int32 * 4),
        ("k_words", c_int32 * 3),
        ("v_words", c_int32),
        ("v_groups", c_int32),
        ("k_sm_page", c_void_p),
    ]


class PackSource(ctypes.Structure):
    """``lf_pack_source``."""

    _fields_ = [("k", c_void_p), ("v", c_void_p), ("stride_b", c_int64), ("stride_h", c_int64),
                ("stride_t", c_int64)]


class DecodeArgs(ctypes.Structure):
    """``lf_decode_args``."""

    _fields_ = [
        ("query", c_void_p), ("q_dtype", c_int32),
        ("k_new", c_void_p), ("v_new", c_void_p),
        ("new_dtype", c_int32),
        ("tail_k", c_void_p), ("tail_v", c_void_p),
        ("tail_dtype", c_int32), ("tail_cap", c_int32),
        ("tail_len", c_void_p),
        ("out", c_void_p), ("out_dtype", c_int32),
        ("n_q", c_int32),
        ("scaling", c_float),
        ("work", c_void_p), ("n_work", c_int32),
        ("seq_work", c_void_p),
        ("workspace", c_void_p), ("workspace_bytes", c_int64),
        ("kernel", c_int32),
        ("q_len", c_int32),
        ("work_host", c_void_p), ("seq_work_host", c_void_p),
        ("commit_new", c_int32),
    ]


_SIGNATURES = {
    "lf_abi_version": (c_int32, []),
    "lf_build_info": (c_char_p, []),
    "lf_status_string": (c_char_p, [c_int32]),
    "lf_pack_pages": (c_int32, [POINTER(PackedLayer), c_void_p, c_void_p, c_int32, c_int64, c_int64, c_int64,
                                c_void_p, c_int32, c_void_p]),
    "lf_pack_pages_multi": (c_int32, [c_void_p, POINTER(PackedLayer), c_void_p, POINTER(PackSource), c_int32,
                                      c_int32, c_void_p, c_int32, c_void_p]),
    "lf_plan_decode": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int32, c_void_p]),
    "lf_decode_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32]),
    "lf_decode_attention": (c_int32, [POINTER(PackedLayer), POINTER(DecodeArgs), c_void_p]),
    "lf_dequantize": (c_int32, [POINTER(PackedLayer), c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "lf_dense_decode_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32]),
    "lf_dense_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                  c_int64, c_int64, c_int64, c_float, c_void_p, c_int32, c_void_p, c_int64,
                                  c_void_p]),
    "lf_asymmetric_codes": (c_int32, [c_void_p, c_int32, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                      c_void_p]),
    "lf_pack_ints": (c_int32, [c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p]),
    "lf_unpack_ints": (c_int32, [c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "lf_decode_attention_noalloc": (c_int32, [POINTER(PackedLayer), POINTER(DecodeArgs), c_void_p]),
    "lf_append_token": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int32,
                                  c_int32, c_int32, c_int32, c_void_p]),
    "lf_noalloc_scratch_bytes": (c_int64, []),
}

ABI_VERSION = 8
_LIB = None


def load() -> ctypes.CDLL:
    """Load the library (once).  Raises ``NativeLibraryMissing`` when it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    import torch  # noqa: F401  -- binds libamdhip64.so.7 to torch's HIP runtime first

    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"{LIB_PATH} is missing: build it with `python -m logitfill_amd.build` "
            "(the packed path has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.lf_abi_version() != ABI_VERSION:
        raise NativeLibraryMissing(f"{LIB_PATH} has ABI {lib.lf_abi_version()}, expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(status: int, call: str) -> None:
    if status != 0:
        msg = load().lf_status_string(status)
        raise LFError(status, msg.decode() if msg else "?", call)


_DTYPE_CODES: dict = {}


def dtype_code(dtype) -> int:
    if not _DTYPE_CODES:
        import torch

        _DTYPE_CODES.update({torch.bfloat16: LF_BF16, torch.float16: LF_FP16, torch.float32: LF_FP32})
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected bfloat16, float16 or float32") from None


def current_stream_ptr(device) -> int:
    """The raw hipStream_t of the current stream on ``device`` (torch's C accessor when this
    build has it: no Stream object per call, which the per-layer decode path would pay twice)."""
    import torch

    index = device.index if isinstance(device, torch.device) else device
    if index is None:
        index = torch.cuda.current_device()
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is not None:
        return int(raw(index))
    return int(torch.cuda.current_stream(index).cuda_stream)


def upload(data, dtype, device):
    """Copy host data (a sequence of numbers, or raw bytes for ``torch.uint8``) to a new device
    tensor without synchronising the host: the data is staged in pinned host memory and copied
    asynchronously on the current stream.  torch's pinned-memory allocator keeps the staging
    block until that copy has run, so the caller may reuse or drop its data at once."""
    import torch

    if isinstance(data, (bytes, bytearray, memoryview)):
        host = torch.frombuffer(bytearray(data), dtype=torch.uint8)
    else:
        host = torch.as_tensor(data, dtype=dtype)
    staged = torch.empty(host.shape, dtype=host.dtype, pin_memory=True)
    staged.copy_(host)
    out = torch.empty(host.shape, dtype=host.dtype, device=device)
    out.copy_(staged, non_blocking=True)
    return out
