"""Backward of the block-sparse masked attention (the reference has none:
gpu/triton_attn.py:9-10, README.md:118).

The gradients of o = softmax(scale q k^T, masked) v are computed from the forward's
output and row log-sum-exp: dV = P^T dO, dP = dO V^T, dS = P (dP - rowsum(dO O)),
dQ = scale dS K, dK = scale dS^T Q, with P = exp(scale q k^T - lse) on live pairs.
``BackwardPlan`` builds the block index at 64 x 64 tiles and its transpose once (on the
device), then every ``backward`` call is one pre-pass and two kernels (pa_attn_bwd).
``SplitBackward`` runs a mask split into disjoint pieces, each in its own basis, the
way the forward's split plan does: the gradients are sums over live pairs, so the
backward of the union is the sum of the pieces' backwards, each taking the whole mask's
lse and rowsum(dO O).
"""
import ctypes

import torch

from . import _lib
from .index import build_device
from .perm import permute_rows, permute_stack, residue_perm
from .spec import DeviceMask, device_mask

TILE = 64
ACCUMULATE = 1   # PA_BWD_ACCUMULATE
DVEC_GIVEN = 2   # PA_BWD_DVEC_GIVEN


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
    evaluate the mask on partial tiles.  residue=s > 1 builds the index in the residue-s
    basis (perm = perm_kv = residue_perm(N, s)), so that ``backward`` can also take the
    tensors in original order and apply the basis in its loads and stores."""

    def __init__(self, mask, N, device=None, perm=None, perm_kv=None, bitmaps=True, residue=0):
        if N % TILE:
            raise ValueError(f"N={N} must be a multiple of {TILE}")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.N, self.device = N, dev
        self.residue = int(residue) if residue and residue > 1 else 0
        if self.residue:
            if perm is not None or perm_kv is not None:
                raise ValueError("residue and perm / perm_kv are exclusive")
            perm = perm_kv = residue_perm(N, self.residue)
        if isinstance(mask, DeviceMask):
            raise ValueError("BackwardPlan takes a mask object (with perm / perm_kv), not a DeviceMask")
        self.dmask = device_mask(mask, N, dev, perm=perm, perm_kv=perm_kv)
        built = build_device(mask, N, TILE, TILE, perm=perm, perm_kv=perm_kv, device=dev, bits=bitmaps)
        kv_idx, kv_num, kv_partial = built[:3]
        self.live = int(built[5])      # live pairs of the mask (per head)
        self.kv_idx, self.kv_num, self.kv_partial = kv_idx.contiguous(), kv_num.contiguous(), kv_partial.contiguous()
        # element bitmaps of the partial tiles, row-major for the dQ pass and transposed for
        # the dK / dV pass, so neither evaluates the mask
        self.kv_bits_off, self.kv_bits = (t.contiguous() for t in built[6]) if bitmaps else (None, None)
        self.q_idx, self.q_num, self.q_partial, self.q_bits_off = transpose_index(
            self.kv_idx, self.kv_num, self.kv_partial, N // TILE, self.kv_bits_off)
        self.q_bits = transpose_bits(self.kv_bits_off, self.kv_bits) if bitmaps else None
        # the dK / dV pass issues the key blocks with the longest lists first
        self.kv_order = torch.argsort(self.q_num, descending=True, stable=True).to(torch.int32).contiguous()

    def backward(self, q, k, v, o, lse, do, scale=None, dq=None, dk=None, dv=None, dvec=None, dvec_given=False,
                 accumulate=False, original_order=False):
        """(dq, dk, dv) for [BH, N, D] f16 / bf16 tensors sharing strides; lse float32 [BH, N]
        from the forward (natural log).  dvec: optional float32 [BH, N] buffer for
        rowsum(dO O) (with dvec_given it already holds it and the pre-pass is skipped).
        accumulate: add the gradients into dq / dk / dv (which must be given).
        original_order (a plan built with residue, D = 128): every array is in original
        order; the kernels read and write through the residue basis."""
        BH, N, D = q.shape
        if N != self.N:
            raise ValueError(f"plan built for N={self.N}, got N={N}")
        ts = (q, k, v, o, do)
        if lse.dtype != torch.float32 or lse.shape != (BH, N) or lse.stride(1) != 1 or lse.stride(0) < N:
            raise ValueError("lse must be float32 [BH, N] with unit column stride and row stride >= N")
        _lib.require_device(*ts, lse)
        for t in ts:
            if t.shape != q.shape or t.dtype != q.dtype or t.stride() != q.stride():
                raise ValueError("q, k, v, o and do must share shape, dtype and strides")
        if q.stride(2) != 1:
            raise ValueError("the last dimension must have unit stride")
        outs = []
        for t, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
            t = torch.empty_like(q) if t is None else t
            if t.shape != q.shape or t.dtype != q.dtype or t.stride() != q.stride():
                raise ValueError(f"{name} must match q in shape, dtype and strides")
            outs.append(t)
        if accumulate and (dq is None or dk is None or dv is None):
            raise ValueError("accumulate needs dq, dk and dv")
        if dvec is None:
            if dvec_given:
                raise ValueError("dvec_given needs dvec")
            # the kernels index dvec with lse's row stride: give it lse's layout
            dvec = torch.empty_strided(lse.shape, lse.stride(), dtype=torch.float32, device=q.device)
        elif dvec.dtype != torch.float32 or dvec.shape != (BH, N) or dvec.stride() != lse.stride():
            raise ValueError("dvec must be float32 [BH, N] with lse's strides")
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
        a.flags = (ACCUMULATE if accumulate else 0) | (DVEC_GIVEN if dvec_given else 0)
        a.kv_order = _lib.ptr(self.kv_order)
        if original_order:
            if not self.residue:
                raise ValueError("original_order needs a plan built with residue")
            a.residue_s = self.residue
        a.mask = self.dmask.struct()
        with torch.cuda.device(q.device):
            _lib.check(_lib.lib().pa_attn_bwd(ctypes.byref(a), _lib.stream_of(q)), "pa_attn_bwd")
        return tuple(outs)


def _fusable(N, s):
    """The residue-s basis can be applied in the backward kernels' loads and stores."""
    per = N // s
    return N % s == 0 and per % 64 == 0 and (per & (per - 1)) == 0


class SplitBackward:
    """The backward of a mask split into disjoint pieces (split.Piece: mask and residue;
    the tile shape is always 64 x 64 here), each piece in its own basis.  Every piece adds
    into the same gradients in original order: at D = 128 a permuted piece reads and
    writes through its residue basis inside the kernels (no copies); otherwise its
    tensors are gathered into the basis and its gradients scattered back, and such pieces
    run first.  Pieces without a live tile are left out."""

    def __init__(self, pieces, N, device=None):
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.N, self.device = N, dev
        order = sorted(pieces, key=lambda p: not (p.residue and p.residue > 1))
        self.steps = []
        for p in order:
            s = int(p.residue) if p.residue and p.residue > 1 else 0
            plan = BackwardPlan(p.mask, N, dev, residue=s)
            if int(plan.kv_num.sum()):
                perm = torch.from_numpy(residue_perm(N, s)).to(dev) if s else None
                self.steps.append((s, perm, plan))

    @property
    def tiles(self):
        return sum(int(plan.kv_num.sum()) for _, _, plan in self.steps)

    @property
    def live(self):
        return sum(plan.live for _, _, plan in self.steps)

    def backward(self, q, k, v, o, lse, do, scale=None):
        """(dq, dk, dv) of the union of the pieces, tensors in the original order."""
        lse = lse.contiguous()
        if not self.steps:
            return tuple(torch.zeros_like(q) for _ in range(3))
        D = q.shape[2]
        outs, dvec, have = None, torch.empty_like(lse), False
        for s, perm, plan in self.steps:
            if s and not (D == 128 and _fusable(self.N, s)):
                (qp, kp, vp, op, dop), _ = permute_stack([q, k, v, o, do], perm, with_positions=False)
                lsep = permute_rows(lse, perm)
                dvp = permute_rows(dvec, perm) if have else torch.empty_like(lsep)
                tgt = permute_stack(list(outs), perm, with_positions=False)[0] if outs is not None else [None] * 3
                g = plan.backward(qp, kp, vp, op, lsep, dop, scale, *tgt, dvec=dvp, dvec_given=have,
                                  accumulate=outs is not None)
                if not have:
                    dvec = permute_rows(dvp, perm, inverse=True)
                outs = permute_stack(list(g), perm, inverse=True, with_positions=False)[0]
            else:
                tgt = outs if outs is not None else (None, None, None)
                outs = plan.backward(q, k, v, o, lse, do, scale, *tgt, dvec=dvec, dvec_given=have,
                                     accumulate=outs is not None, original_order=bool(s))
            have = True
        return tuple(outs)
