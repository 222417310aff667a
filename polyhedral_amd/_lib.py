"""ctypes binding of libpolyattn_amd.so, the C ABI declared in include/polyattn_amd.h.

There is no fallback: if the library is missing, or a tensor is not on a HIP
device, the call raises.  The library is loaded after ``import torch`` so that
it binds to the HIP runtime torch already loaded.
"""
import ctypes
import pathlib

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libpolyattn_amd.so"

PA_OK, PA_E_INVALID, PA_E_HIP, PA_E_UNSUPPORTED = 0, -1, -2, -3
PA_F32, PA_F16, PA_BF16 = 0, 1, 2
MAX_TERMS = 8
ABI_VERSION = 19

c_i32, c_i64, c_f32, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p


class PaTerm(ctypes.Structure):
    _fields_ = [("kind", c_i32), ("p0", c_i32), ("p1", c_i32), ("p2", c_i32)]


class PaMask(ctypes.Structure):
    _fields_ = [("n_include", c_i32), ("n_exclude", c_i32), ("terms", PaTerm * MAX_TERMS),
                ("perm_q", c_vp), ("perm_kv", c_vp), ("dense_bits", c_vp), ("dense_words", c_i64)]


class PaAttnArgs(ctypes.Structure):
    _fields_ = [("q", c_vp), ("k", c_vp), ("v", c_vp), ("o", c_vp),
                ("q_sb", c_i64), ("q_sn", c_i64), ("k_sb", c_i64), ("k_sn", c_i64),
                ("v_sb", c_i64), ("v_sn", c_i64), ("o_sb", c_i64), ("o_sn", c_i64),
                ("BH", c_i64), ("N", c_i64), ("D", c_i32), ("dtype", c_i32), ("scale", c_f32),
                ("BQ", c_i32), ("A", c_i32),
                ("kv_idx", c_vp), ("kv_num", c_vp), ("kv_partial", c_vp), ("kv_wave_bits", c_vp),
                ("pitch", c_i64), ("kv_bits_off", c_vp), ("kv_bits", c_vp), ("mask", PaMask),
                ("gather_q", c_i32), ("gather_kv", c_i32), ("scatter_o", c_i32),
                ("residue_s", c_i32), ("residue_qlog2", c_i32),
                ("lse", c_vp), ("lse_sb", c_i64),
                ("prev_o", c_vp), ("prev_dtype", c_i32), ("prev_sb", c_i64), ("prev_sn", c_i64),
                ("prev_lse", c_vp), ("qblock_order", c_vp), ("kv_steps", c_vp), ("steps_pitch", c_i64),
                ("heads_desc", c_i32), ("gather_mult", c_i32), ("gather_scatter", c_i32), ("wsel", c_vp),
                ("wsel_sb", c_i64), ("run_steps", c_vp), ("run_start", c_vp), ("run_groups", c_i32),
                ("wave_split", c_i32)]


class PaSplitArgs(ctypes.Structure):
    _fields_ = [("first", ctypes.POINTER(PaAttnArgs)), ("second", ctypes.POINTER(PaAttnArgs)),
                ("run_steps", c_vp), ("run_start", c_vp), ("run_groups", c_i32), ("kv_bits", c_vp),
                ("sync", c_vp), ("sync_groups", c_i32), ("sync_signal", c_i32), ("sync_wait", c_i32),
                ("status", c_vp), ("items", c_vp), ("n_items", c_i64)]


class PaDecodeArgs(ctypes.Structure):
    _fields_ = [("q", c_vp), ("q_sb", c_i64), ("q_sn", c_i64), ("nq", c_i32), ("qpos0", c_i64),
                ("k_cache", c_vp), ("v_cache", c_vp), ("c_sb", c_i64), ("c_sn", c_i64),
                ("capacity", c_i64), ("length", c_i64), ("residue_s", c_i32), ("mask", PaMask),
                ("BH", c_i64), ("D", c_i32), ("dtype", c_i32), ("scale", c_f32),
                ("o", c_vp), ("o_sb", c_i64), ("o_sn", c_i64), ("lse", c_vp), ("lse_sb", c_i64),
                ("workspace", c_vp), ("workspace_bytes", c_i64), ("k_new", c_vp), ("v_new", c_vp),
                ("new_sb", c_i64), ("new_sn", c_i64), ("n_new", c_i64), ("new_pos0", c_i64)]


class PaAttnBwdArgs(ctypes.Structure):
    _fields_ = [("q", c_vp), ("k", c_vp), ("v", c_vp), ("o", c_vp), ("dout", c_vp),
                ("dq", c_vp), ("dk", c_vp), ("dv", c_vp), ("sb", c_i64), ("sn", c_i64),
                ("lse", c_vp), ("dvec", c_vp), ("lse_sb", c_i64), ("BH", c_i64), ("N", c_i64),
                ("D", c_i32), ("dtype", c_i32), ("scale", c_f32),
                ("kv_idx", c_vp), ("kv_num", c_vp), ("kv_partial", c_vp), ("pitch", c_i64),
                ("q_idx", c_vp), ("q_num", c_vp), ("q_partial", c_vp), ("tpitch", c_i64),
                ("kv_bits_off", c_vp), ("kv_bits", c_vp), ("q_bits_off", c_vp), ("q_bits", c_vp), ("flags", c_i32), ("residue_s", c_i32), ("kv_order", c_vp),
                ("mask", PaMask)]


# name -> (restype, argtypes); every symbol of include/polyattn_amd.h
SIGNATURES = {
    "pa_last_error": (ctypes.c_char_p, []),
    "pa_abi_version": (c_i32, []),
    "pa_index_classify": (ctypes.c_int, [ctypes.POINTER(PaMask), c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_vp]),
    "pa_index_compact": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i64, c_vp]),
    "pa_index_bits": (ctypes.c_int, [ctypes.POINTER(PaMask), c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i64, c_vp,
                                     c_vp, c_vp, c_vp]),
    "pa_index_steps": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp,
                                      c_vp, c_i64, c_vp]),
    "pa_index_run": (ctypes.c_int, [ctypes.POINTER(c_vp), ctypes.POINTER(c_i64), ctypes.POINTER(c_i32), c_i32, c_i64,
                                    c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp]),
    "pa_attn_fwd_split": (ctypes.c_int, [ctypes.POINTER(PaSplitArgs), c_vp]),
    "pa_permute_rows": (ctypes.c_int, [c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                       c_i32, c_vp]),
    "pa_permute_stack": (ctypes.c_int, [c_vp, c_vp, c_i32, c_vp, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64, c_i64,
                                        c_vp, c_vp, c_i32, c_vp]),
    "pa_invert_perm": (ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    "pa_residue_perm": (ctypes.c_int, [c_vp, c_i64, c_i32, c_vp]),
    "pa_attn_fwd": (ctypes.c_int, [ctypes.POINTER(PaAttnArgs), c_vp]),
    "pa_lse_merge": (ctypes.c_int, [ctypes.POINTER(c_vp), ctypes.POINTER(c_vp), c_i32, c_vp, c_i32, c_vp,
                                    c_i64, c_i64, c_i32, c_vp]),
    "pa_kv_append": (ctypes.c_int, [c_vp, c_vp, c_i64, c_i64, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32,
                                    c_i64, c_i64, c_i32, c_vp]),
    "pa_decode_workspace": (ctypes.c_int, [ctypes.POINTER(PaDecodeArgs), ctypes.POINTER(c_i64)]),
    "pa_decode_fwd": (ctypes.c_int, [ctypes.POINTER(PaDecodeArgs), c_vp]),
    "pa_decode_fwd_static": (ctypes.c_int, [ctypes.POINTER(PaDecodeArgs), c_vp]),
    "pa_index_transpose": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i32, c_i64, c_i32, c_vp, c_vp, c_vp, c_vp, c_i64,
                                          c_vp]),
    "pa_index_bits_transpose": (ctypes.c_int, [c_vp, c_i32, c_i64, c_vp, c_vp, c_vp]),
    "pa_attn_bwd": (ctypes.c_int, [ctypes.POINTER(PaAttnBwdArgs), c_vp]),
}

_LIB = None


class PolyattnError(RuntimeError):
    """A C-ABI call returned an error status."""


def lib():
    """The loaded library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m polyhedral_amd.build` "
                               "(there is no non-HIP fallback)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        if handle.pa_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI version {handle.pa_abi_version()} != {ABI_VERSION}; rebuild")
        _LIB = handle
    return _LIB


def check(rc, what):
    if rc != PA_OK:
        msg = lib().pa_last_error().decode(errors="replace")
        kind = {PA_E_INVALID: "invalid argument", PA_E_HIP: "HIP error",
                PA_E_UNSUPPORTED: "unsupported"}.get(rc, f"status {rc}")
        raise PolyattnError(f"{what}: {kind}: {msg}")


def require_device(*tensors):
    """Every tensor must live on a HIP device: the kernels have no host path."""
    for t in tensors:
        if t is not None and (not isinstance(t, torch.Tensor) or t.device.type != "cuda"):
            dev = t.device if isinstance(t, torch.Tensor) else type(t).__name__
            raise RuntimeError(f"polyhedral_amd kernels run on the GPU only; got a tensor on {dev}")


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(None)


DTYPE_CODE = {torch.float32: PA_F32, torch.float16: PA_F16, torch.bfloat16: PA_BF16}


def dtype_code(t):
    try:
        return DTYPE_CODE[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, float16 or bfloat16") from None
