"""Class-A re-indexing: the call surface of gpu/permute.py, with the copies on the GPU.

residue_perm / identity_perm return host int32 arrays exactly as gpu/permute.py:12-19
does (drivers upload them with torch.from_numpy(...).cuda()); the residue order is
built in O(N) as the concatenation of the classes c = 0..s-1, each in increasing
position -- the stable sort by (i mod s, i div s).  apply_perm and invert run the
pa_permute_rows / pa_invert_perm kernels.
"""
import numpy as np
import torch

from . import _lib


def residue_perm(N, s):
    """Permuted position p -> original position, grouping positions by i mod s."""
    return np.concatenate([np.arange(c, N, s) for c in range(s)]).astype(np.int32)


def identity_perm(N):
    return np.arange(N, dtype=np.int32)


def _perm32(perm, device):
    if not isinstance(perm, torch.Tensor):
        perm = torch.from_numpy(np.asarray(perm, dtype=np.int32))
    return perm.to(device=device, dtype=torch.int32).contiguous()


def permute_rows(x, perm, inverse=False, out=None):
    """Row gather out[:, p] = x[:, perm[p]] (or scatter out[:, perm[p]] = x[:, p]) on dim 1."""
    _lib.require_device(x)
    if x.dim() < 2:
        raise ValueError("permute_rows expects [BH, N, ...]")
    if x.stride(-1) != 1 or not x[0, 0].is_contiguous():
        x = x.contiguous()
    BH, N = x.shape[0], x.shape[1]
    p = _perm32(perm, x.device)
    if p.numel() != N:
        raise ValueError(f"perm has {p.numel()} entries for {N} rows")
    if out is None:
        out = torch.empty_like(x, memory_format=torch.contiguous_format)
    esz = x.element_size()
    row_bytes = x[0, 0].numel() * esz
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().pa_permute_rows(_lib.ptr(x), _lib.ptr(out), _lib.ptr(p), BH, N, row_bytes,
                                              x.stride(0) * esz, x.stride(1) * esz,
                                              out.stride(0) * esz, out.stride(1) * esz, int(inverse),
                                              _lib.stream_of(x)), "pa_permute_rows")
    return out


def permute_stack(tensors, perm, positions=None, inverse=False, with_positions=True):
    """One launch (pa_permute_stack): every tensor of `tensors` ([BH, N, ...], one shape)
    gathered through perm (out[:, p] = x[:, perm[p]]; inverse=True scatters), and the
    position ids moved with the tokens: pos_out[p] = positions[perm[p]] (positions None:
    the original positions perm[p] themselves).  Returns (list of tensors, int64 [N]
    positions or None).  The permuted stack then runs a whole forward in the permuted
    basis, and position-dependent ops (RoPE) read pos_out instead of arange(N)
    (gpu/exp5_amortisation.py:44-57, 89-118)."""
    tensors = list(tensors)
    if not 1 <= len(tensors) <= 8:
        raise ValueError("permute_stack takes 1 to 8 tensors")
    _lib.require_device(*tensors)
    x0 = tensors[0]
    if x0.dim() < 2:
        raise ValueError("permute_stack expects [BH, N, ...] tensors")
    xs = [x if (x.stride(-1) == 1 and x[0, 0].is_contiguous()) else x.contiguous() for x in tensors]
    for x in xs[1:]:
        if x.shape != x0.shape or x.dtype != x0.dtype or x.stride() != xs[0].stride() or x.device != x0.device:
            raise ValueError("permute_stack tensors must share shape, dtype, strides and device")
    BH, N = x0.shape[0], x0.shape[1]
    p = _perm32(perm, x0.device)
    if p.numel() != N:
        raise ValueError(f"perm has {p.numel()} entries for {N} rows")
    outs = [torch.empty_like(x, memory_format=torch.contiguous_format) for x in xs]
    pos_in = None
    if positions is not None:
        pos_in = positions.to(device=x0.device, dtype=torch.int64).contiguous()
        if pos_in.numel() != N:
            raise ValueError(f"positions has {pos_in.numel()} entries for {N} rows")
    pos_out = torch.empty(N, dtype=torch.int64, device=x0.device) if with_positions else None
    esz = x0.element_size()
    row_bytes = xs[0][0, 0].numel() * esz
    n = len(xs)
    srcs = (_lib.c_vp * n)(*[x.data_ptr() for x in xs])
    dsts = (_lib.c_vp * n)(*[o.data_ptr() for o in outs])
    with torch.cuda.device(x0.device):
        _lib.check(_lib.lib().pa_permute_stack(srcs, dsts, n, _lib.ptr(p), BH, N, row_bytes,
                                               xs[0].stride(0) * esz, xs[0].stride(1) * esz,
                                               outs[0].stride(0) * esz, outs[0].stride(1) * esz,
                                               _lib.ptr(pos_in), _lib.ptr(pos_out), int(inverse),
                                               _lib.stream_of(x0)), "pa_permute_stack")
    return outs, pos_out


def apply_perm(x, perm):
    """gpu/permute.py:22-24: x [BH, N, D] -> rows reordered so position p holds original perm[p]."""
    return permute_rows(x, perm, inverse=False)


def invert(perm):
    """gpu/permute.py:27-31: inv[perm[p]] = p, same dtype and device as perm."""
    _lib.require_device(perm)
    p = perm.to(torch.int32).contiguous()
    inv = torch.empty_like(p)
    with torch.cuda.device(p.device):
        _lib.check(_lib.lib().pa_invert_perm(_lib.ptr(p), _lib.ptr(inv), p.numel(), _lib.stream_of(p)),
                   "pa_invert_perm")
    return inv.to(perm.dtype)


def residue_perm_device(N, s, device="cuda"):
    """The residue permutation computed on the device (closed form), int32 [N]."""
    out = torch.empty(N, dtype=torch.int32, device=device)
    _lib.require_device(out)
    with torch.cuda.device(out.device):
        _lib.check(_lib.lib().pa_residue_perm(_lib.ptr(out), N, s, _lib.stream_of(out)), "pa_residue_perm")
    return out


def permutation_cost_ms(q, k, v, perm, reps=50):
    """gpu/permute.py:34-38: the one-time cost of permuting Q, K and V, reported separately."""
    from .timing import time_ms
    return time_ms(lambda: (apply_perm(q, perm), apply_perm(k, perm), apply_perm(v, perm)), reps=reps)[0]
