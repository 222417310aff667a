"""Backward of the block-sparse masked attention (the reference has none:
gpu/triton_attn.py:9-10, README.md:118).

The gradients of o = softmax(scale q k^T, masked) v are computed from the forward's
output and row log-sum-exp: dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO O)),
dQ = scale dS K, dK = scale dS^T Q, with P = exp(scale q k^T - lse) on live pairs.
``BackwardPlan`` builds the block index at 64 x 64 tiles and its transpose once (on the
device), then every ``backward`` call is one pre-pass and two kernels (pa_attn_bwd).
"""
import ctypes

import torch

from . import _lib
from .index import build_device
from .spec import DeviceMask, device_mask

TILE = 64


def transpose_index(kv_idx, kv_num, kv_partial, n_kv_blocks, kv_bits_off=None):
    """Per key block, the query blocks whose list holds it (ascending) and the partial
    flags: (q_idx int32 [nk, tpitch], q_num int32 [nk], q_partial int8 [nk, tpitch],
    q_bits_off int32 [nk, tpitch] or None).  With kv_bits_off (pa_index_bits of the same
    index), q_bits_off holds each tile's bitmap offset (-1 for a full tile)."""
    _lib.require_device(kv_idx, kv_num, kv_partial)
    dev = kv_num.device
    nq, pitch = kv_idx.shape
    q_num = torch.empty(n_kv_blocks, dtype=torch.int32, device=dev)
    L = _lib.lib()
    bo = _lib.ptr(kv_bits_off) if kv_bits_off is not None else None
    with torch.cuda.device(dev):
        st = _lib.stream_of(q_num)
        _lib.check(L.pa_index_transpose(_lib.ptr(kv_idx), _lib.ptr(kv_num), _lib.ptr(kv_partial), bo, nq, pitch,
                                        n_kv_blocks, _lib.ptr(q_num), None, None, None, 0, st), "pa_index_transpose")
        tp = int(q_num.max().item()) if n_kv_blocks else 0
        q_idx = torch.zeros((n_kv_blocks, max(tp, 1)), dtype=torch.int32, device=dev)
        q_partial = torch.zeros((n_kv_blocks, max(tp, 1)), dtype=torch.int8, device=dev)
        q_bits_off = torch.full((n_kv_blocks, max(tp, 1)), -1, dtype=torch.int32, device=dev) if bo else None
        if tp:
            _lib.check(L.pa_index_transpose(_lib.ptr(kv_idx), _lib.ptr(kv_num), _lib.ptr(kv_partial), bo, nq, pitch,
                                            n_kv_blocks, _lib.ptr(q_num), _lib.ptr(q_idx), _lib.ptr(q_partial),
                                            _lib.ptr(q_bits_off) if bo else None, q_idx.shape[1], st),
                       "pa_index_transpose")
    return q_idx, q_num, q_partial, q_bits_off


def transpose_bits(kv_bits_off, kv_bits):
    """The partial tiles' bitmaps (pa_index_bits at 64 x 64, row-major) transposed to
    column-major at the same offsets."""
    _lib.require_device(kv_bits_off, kv_bits)
    q_bits = torch.zeros_like(kv_bits)
    nq, pitch = kv_bits_off.shape
    with torch.cuda.device(kv_bits.device):
        _lib.check(_lib.lib().pa_index_bits_transpose(_lib.ptr(kv_bits_off), nq, pitch, _lib.ptr(kv_bits),
                                                       _lib.ptr(q_bits), _lib.stream_of(q_bits)),
                   "pa_index_bits_transpose")
    return q_bits


class BackwardPlan:
    """The 64 x 64 block index of `mask` at length N (and its transpose), built once.
    perm / perm_kv: index-space position -> original position, when the tensors given to
    ``backward`` are relabelled (the mask is evaluated in original coordinates).
    bitmaps=False leaves out the partial tiles' element bitmaps: the kernels then
    evaluate the mask on partial tiles."""

    def __init__(self, mask, N, device=None, perm=None, perm_kv=None, bitmaps=True):
        if N % TILE:
            raise ValueError(f"N={N} must be a multiple of {TILE}")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.N, self.device = N, dev
        if isinstance(mask, DeviceMask):
            raise ValueError("BackwardPlan takes a mask object (with perm / perm_kv), not a DeviceMask")
        self.dmask = device_mask(mask, N, dev, perm=perm, perm_kv=perm_kv)
        built = build_device(mask, N, TILE, TILE, perm=perm, perm_kv=perm_kv, device=dev, bits=bitmaps)
        kv_idx, kv_num, kv_partial = built[:3]
        self.kv_idx, self.kv_num, self.kv_partial = kv_idx.contiguous(), kv_num.contiguous(), kv_partial.contiguous()
        # element bitmaps of the partial tiles, row-major for the dQ pass and transposed for
        # the dK / dV pass, so neither evaluates the mask
        self.kv_bits_off, self.kv_bits = (t.contiguous() for t in built[6]) if bitmaps else (None, None)
        self.q_idx, self.q_num, self.q_partial, self.q_bits_off = transpose_index(
            self.kv_idx, self.kv_num, self.kv_partial, N // TILE, self.kv_bits_off)
        self.q_bits = transpose_bits(self.kv_bits_off, self.kv_bits) if bitmaps else None

    def backward(self, q, k, v, o, lse, do, scale=None, dq=None, dk=None, dv=None):
        """(dq, dk, dv) for [BH, N, D] f16 / bf16 tensors sharing strides; lse float32 [BH, N]
        from the forward (natural log)."""
        BH, N, D = q.shape
        if N != self.N:
            raise ValueError(f"plan built for N={self.N}, got N={N}")
        ts = (q, k, v, o, do)
        _lib.require_device(*ts, lse)
        for t in ts:
            if t.shape != q.shape or t.dtype != q.dtype or t.stride() != q.stride():
                raise ValueError("q, k, v, o and do must share shape, dtype and strides")
        if q.stride(2) != 1:
            raise ValueError("the last dimension must have unit stride")
        if lse.dtype != torch.float32 or lse.shape != (BH, N) or lse.stride(1) != 1:
            raise ValueError("lse must be float32 [BH, N] with unit row stride")
        outs = []
        for t, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            t = torch.empty_like(q) if t is None else t
            if t.shape != q.shape or t.dtype != q.dtype or t.stride() != q.stride():
                raise ValueError(f"{name} must match q in shape, dtype and strides")
            outs.append(t)
        dvec = torch.empty((BH, N), dtype=torch.float32, device=q.device)
        a = _lib.PaAttnBwdArgs()
        a.q, a.k, a.v, a.o, a.dout = (_lib.ptr(t) for t in ts)
        a.dq, a.dk, a.dv = (_lib.ptr(t) for t in outs)
        a.sb, a.sn = q.stride(0), q.stride(1)
        a.lse, a.dvec, a.lse_sb = _lib.ptr(lse), _lib.ptr(dvec), lse.stride(0)
        a.BH, a.N, a.D, a.dtype = BH, N, D, _lib.dtype_code(q)
        a.scale = float(scale) if scale else float(D ** -0.5)
        a.kv_idx, a.kv_num, a.kv_partial = _lib.ptr(self.kv_idx), _lib.ptr(self.kv_num), _lib.ptr(self.kv_partial)
        a.pitch = self.kv_idx.shape[1]
        a.q_idx, a.q_num, a.q_partial = _lib.ptr(self.q_idx), _lib.ptr(self.q_num), _lib.ptr(self.q_partial)
        a.tpitch = self.q_idx.shape[1]
        if self.kv_bits is not None:
            a.kv_bits_off, a.kv_bits = _lib.ptr(self.kv_bits_off), _lib.ptr(self.kv_bits)
            a.q_bits_off, a.q_bits = _lib.ptr(self.q_bits_off), _lib.ptr(self.q_bits)
        a.mask = self.dmask.struct()
        with torch.cuda.device(q.device):
            _lib.check(_lib.lib().pa_attn_bwd(ctypes.byref(a), _lib.stream_of(q)), "pa_attn_bwd")
        return tuple(outs)

