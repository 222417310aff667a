"""Disjoint split + log-sum-exp merge (no counterpart in the reference's gpu/)."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.split import Piece, SplitPlan, lse_merge  # noqa: E402,F401
