"""Kernel-level API (mirrors the reference's ``dcr_attention.kernel``)."""
