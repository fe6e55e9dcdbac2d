"""CPU oracle for the packed decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy float32 arithmetic, the reference algorithm of
LogitFill's ``logitfill.packed`` backend:

* ``oracle.layout``    -- tier tables, asymmetric min-max codes, LSB-first int32
  packing, the Key/Value page packers and the dense dequantisers
  (reference ``src/logitfill/packed/layout.py:12-182``);
* ``oracle.history``   -- the per-layer page store: flush trigger and the
  concatenation axes of the packed history
  (reference ``src/logitfill/packed/cache.py:48-90``);
* ``oracle.attention`` -- the dense dequantise-then-attend decode path
  (reference ``src/logitfill/packed/reference.py:10-56``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from here, and only as the checker or the
timed CPU baseline.  The product (``logitfill_amd``) never imports it: every
product call runs the HIP kernels and fails loudly when they are missing.

Pinning status (each function is checked by ``tests/test_oracle_*.py`` against
hand-computed known answers, invariants, brute force on tiny inputs and the
reference's own tests restated):

* tier_tables, asymmetric_codes, pack_ints/unpack_ints, quantize_key_page,
  quantize_value_page, dequantize_key/value, LayerHistory, reference_attention:
  pinned.  No function here is "parity unpinned".
"""
