"""gpu/launchsweep.py call surface: LAUNCH, _HARD_FLOOR, _warn_if_on_boundary."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.launch import LAUNCH, _HARD_FLOOR, _warn_if_on_boundary  # noqa: E402,F401
