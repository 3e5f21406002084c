"""Kernel-backed ops (module path mirrors the reference's ``kernels`` package)."""
