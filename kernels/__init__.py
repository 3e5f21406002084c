"""The reference's import path for the attention ops (``kernels.flash_attn``), served by
the HIP library in ``tinytrain_amd``."""
