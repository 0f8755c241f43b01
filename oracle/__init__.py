"""CPU oracle for the packed-INT2 RoLaQ MLA cache path.

TEST INFRASTRUCTURE ONLY. This package is the checker: it is imported by
``tests/``, by ``__graft_entry__.smoke()`` and by the ``cpu_baseline`` leg of
``bench.py``, and by nothing else. The product path (``mla_kv_quant_amd``)
never imports it and fails loudly when its HIP library is missing.

Each function restates a piece of the reference (noforit/mla_kv_quant) and
cites the file:line it follows. Floating-point parts use torch on the CPU in
the same operation order as the reference, so that the oracle reproduces the
reference bit for bit on the machine it runs on; byte/integer parts use numpy.

Pinning (what checks each function, see ``tests/test_oracle_*.py``):

* ``codec.lloyd_codec`` -- golden vectors written by importing the reference's
  ``mla_quant.oscar.oscar_lloyd_int2_qdq`` (``tests/golden/make_golden.py``),
  plus closed forms (constant group, +-1 alternating group, 4-level property,
  monotonicity).
* ``codec.rotate_quantize`` -- golden vectors from the reference's
  ``mla_quant.quantizer.rotate_quantize``; rotation-orthogonality identities.
* ``codec.signal_gain`` -- closed form ``train.py:21-29`` evaluated in float64
  and the bound ``g(t_max) = 1.3``.
* ``layout.pack_codes`` / ``unpack_codes`` -- the byte layout is defined by this
  build (the reference's packer lives in an un-vendored SGLang fork); pinned by
  round trips, an independent bit-by-bit packer and hand-written vectors.
* ``window`` -- brute force over tiny sequences against the HF cache's
  positional sink/recent rule, and golden transitions from the reference's
  ``FakeQuantizedDynamicCache``.
* ``attention`` -- float64 brute force on tiny inputs, exact-softmax
  invariants (split-K LSE merge equals the unsplit result, empty splits are
  neutral) and rotation invariance of the absorbed form.
"""

from . import codec, layout, window, attention  # noqa: F401
