"""``kernels.flash_attn`` as the reference's callers import it (model.py:6,
tests/test_flash_attn.py:4): the same names, backed by libttfa.so.

The objects are those of ``tinytrain_amd.kernels.flash_attn`` (the ops are registered once,
under ``tinytrain::flash_attn_fwd`` / ``tinytrain::flash_attn_bwd``), so a caller that
imports either path gets the same custom ops.  ``flash_attn_varlen*`` and the decode op are
additions with no reference counterpart.
"""

from tinytrain_amd.kernels.flash_attn import (  # noqa: F401
    FlashAttnInputError,
    _backward,
    _forward,
    flash_attn,
    flash_attn_bwd,
    flash_attn_fwd,
    flash_attn_varlen,
    flash_attn_varlen_bwd,
    flash_attn_varlen_fwd,
)

__all__ = ["_forward", "_backward", "flash_attn", "flash_attn_fwd", "flash_attn_bwd",
           "flash_attn_varlen", "flash_attn_varlen_fwd", "flash_attn_varlen_bwd",
           "FlashAttnInputError"]
