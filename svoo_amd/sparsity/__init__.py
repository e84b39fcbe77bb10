"""Offline sparsity profiles consumed by the online mask (per step, layer and head)."""

from .lookup import SparsityLookup

__all__ = ["SparsityLookup"]
