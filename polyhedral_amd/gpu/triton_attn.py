"""gpu/triton_attn.py call surface (the name is kept; the kernel is HIP, not Triton)."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.attention import (CAUSAL, DILATED, LOCAL_STRIDED, PREFIX_LM, SINKS,  # noqa: E402,F401
                                      TWOBAND, WINDOW, _PIPELINE_FALLBACK, _assert_kinds_match,
                                      block_sparse_attention)
