"""gpu/bench.py call surface: time_ms, paired_time, report."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.timing import paired_time, report, time_ms  # noqa: E402,F401
