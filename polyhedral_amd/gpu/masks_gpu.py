"""gpu/masks_gpu.py call surface: kind constants, SPECS, numpy_mask, triton_params,
flex_mask_mod, dense_bool, check_agreement."""
import os as _os
import sys as _sys

_ROOT = _os.path.dirname(_os.path.dirname(_os.path.dirname(_os.path.abspath(__file__))))
if _ROOT not in _sys.path:
    _sys.path.insert(0, _ROOT)

from polyhedral_amd.registry import (CAUSAL, DILATED, LOCAL_STRIDED, PREFIX_LM, SINKS, SPECS,  # noqa: E402,F401
                                     TWOBAND, WINDOW, check_agreement, dense_bool, flex_mask_mod,
                                     numpy_mask, triton_params)
