"""Counterpart of the reference's polyattn package for the attention hot path:
``masks`` (the predicate zoo) and ``cost`` (the element-count model) only."""
from . import cost, masks  # noqa: F401
