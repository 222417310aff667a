"""gpu/blockindex.py call surface: BlockIndex, build, to_cuda (built on the GPU)."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.index import BlockIndex, build, build_device, to_cuda, wave_bits_for  # noqa: E402,F401
