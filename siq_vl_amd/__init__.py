"""MI355X-native (gfx950) SiQ-VL training hot path.

* ``siq_vl_amd.attention`` -- varlen packed flash attention (fwd/bwd), the
  ``siq_varlen`` transformers attention backend and the FA-style varlen op.
* ``siq_vl_amd.cross_entropy`` -- fused lm_head linear + cross-entropy.
* ``siq_vl_amd.collator`` -- packing collator (cu_seqlens batches).
* ``siq_vl_amd.text_model`` -- the fused-CE forward for SiQ-VL's text model.

All compute runs in hand-written HIP kernels behind the C ABI of
``include/siq_kernels.h`` (``libsiq_kernels.so``, built in-tree).
"""

__version__ = "0.1.0"
