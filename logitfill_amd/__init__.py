"""MI355X-native (gfx950) LogitFill packed decode path.

``logitfill_amd.packed`` mirrors the reference's ``logitfill.packed`` backend:
the packed-cache object, the page-compress call and the decode-attention call,
backed by hand-written HIP kernels in ``liblogitfill_amd.so`` (C ABI in
``include/logitfill_amd.h``).
"""

__version__ = "0.1.0"
