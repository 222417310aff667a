"""Counterpart of the reference's polyattn package for the attention hot path:
``masks`` (the predicate zoo), ``cost`` (the element-count model) and, of
``transforms``, the per-tile key-row count ``kv_per_tile`` that the traffic driver
imports."""
from . import cost, masks, transforms  # noqa: F401
