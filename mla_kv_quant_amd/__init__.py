"""MI355X-native packed-INT2 RoLaQ MLA cache path.

Hand-written HIP kernels for gfx950 behind a C ABI (``include/rolaq_mla.h``,
``librolaq_mla.so``), reached from PyTorch through ``ctypes``:

* ``writer.try_fast_decode_store`` / ``writer.write_prefill`` /
  ``writer.scatter_pack_rows`` -- fused rotate + Lloyd INT2 quantize + pack +
  rope / BF16-window stores;
* ``decode.prepare_gf_splits`` / ``decode.packed_mla_decode_gf_fwd`` -- absorbed
  MLA decode over the packed cache with split-K and LSE merge;
* ``extend.packed_mla_extend_fwd`` -- causal chunked-prefill attention over the
  packed prefix plus the chunk;
* ``artifacts`` -- RoLaQ artifact loading and read-rotation folding.

The library is loaded lazily on first use and there is no CPU fallback.
"""

from . import artifacts, kernels, synth  # noqa: F401
from .pool import PackedMLAPool  # noqa: F401

__all__ = ["artifacts", "kernels", "synth", "PackedMLAPool"]
