"""gpu/permute.py call surface: residue_perm, identity_perm, apply_perm, invert, permutation_cost_ms."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.perm import (apply_perm, identity_perm, invert, permutation_cost_ms,  # noqa: E402,F401
                                 permute_rows, residue_perm, residue_perm_device)
