"""MI355X (gfx950) causal GQA FlashAttention for the tinytrain training stack.

* ``tinytrain_amd.kernels.flash_attn`` -- the ``tinytrain::flash_attn_fwd/_bwd`` custom
  ops and ``flash_attn``, backed by the hand-written HIP library libttfa.so.
* ``tinytrain_amd.attention`` -- the model-side ``attn_impl`` switch (``"sdpa"`` or
  ``"hip"``).
* ``tinytrain_amd.build`` -- the gfx950 hipcc build of libttfa.so.
"""

__version__ = "0.1.0"
