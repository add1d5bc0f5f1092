"""Packed prefill metadata (the inputs of the paged prefill path)."""

from .batch import PrefillBatch

__all__ = ["PrefillBatch"]
