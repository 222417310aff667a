"""gpu/reference.py call surface: attention_reference, max_abs_err (dense torch)."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.dense import attention_reference, max_abs_err  # noqa: E402,F401
