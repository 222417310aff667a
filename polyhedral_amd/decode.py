"""Decoding against a key / value cache kept in a class-A basis.

The reference relabels tokens once per forward for prefill and leaves decoding open:
new keys arrive in original order and "would have to be inserted at permuted
positions" (docs/NOTES.md:2145-2153, 2201-2203).  A cache of fixed capacity C (a
multiple of s) in the residue-s basis of gpu/permute.py:12-15 answers it: every class
owns a segment of C / s rows and the token at original position t sits at row
(t mod s) (C / s) + t div s, the end of its class's segment, so appending writes one
row per token and tensor and never moves a cached row (``pa_kv_append``).  Attention
of the newest query rows to the cache (``pa_decode_fwd``) reads only the live keys'
rows, in either basis; the relabelling makes live keys contiguous, so it visits fewer
blocks.  s = 1 (residue 0 or 1) is the identity basis.
"""
import ctypes

import numpy as np
import torch

from . import _lib
from .spec import DeviceMask, device_mask

MAX_QUERIES = 8


def basis_rows(t, residue, capacity):
    """Cache rows of original positions t: (t mod s) (capacity / s) + t div s."""
    s = int(residue) if residue and residue > 1 else 1
    t = np.asarray(t, dtype=np.int64)
    return (t % s) * (capacity // s) + t // s


def _rows_ok(t, name):
    if t.dim() != 3 or t.stride(2) != 1:
        raise ValueError(f"{name} must be [BH, n, D] with unit stride in the last dimension")


class DecodeLaunch:
    """A validated pa_decode_fwd call with its workspace (or a pa_decode_fwd_static call,
    which uses the library's scratch); __call__ launches it on the current stream of its
    device and returns the output."""

    def __init__(self, args, keep, out, device, static_scratch=False):
        self.args, self.keep, self.out, self.device = args, keep, out, device
        self.entry = "pa_decode_fwd_static" if static_scratch else "pa_decode_fwd"
        self._fn = getattr(_lib.lib(), self.entry)
        self._ref = ctypes.byref(args)

    def __call__(self):
        _lib.check(self._fn(self._ref, _lib.stream_of(self.out)), self.entry)
        return self.out


# classes of the largest residue basis a cache may use (the library's limit too)
MAX_CLASSES = 4096
# size of the library's per-GPU scratch that pa_decode_fwd_static writes its partials to
STATIC_SCRATCH_BYTES = 8 << 20


class KVCache:
    """Keys and values of BH heads, capacity rows each, in the residue-``residue`` basis."""

    def __init__(self, BH, capacity, D, dtype=torch.bfloat16, residue=0, device=None):
        s = int(residue) if residue and residue > 1 else 1
        if s > MAX_CLASSES:
            raise ValueError(f"residue={residue}: a cache's basis has at most {MAX_CLASSES} classes")
        if capacity < 1 or capacity % s:
            raise ValueError(f"capacity={capacity} must be a positive multiple of the residue stride {s}")
        dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.k = torch.zeros(BH, capacity, D, dtype=dtype, device=dev)
        self.v = torch.zeros_like(self.k)
        self.BH, self.capacity, self.D, self.residue, self.device = BH, capacity, D, s, dev
        self.length = 0

    def rows(self, t):
        """Cache rows of original positions t."""
        return basis_rows(t, self.residue, self.capacity)

    def _check_new(self, k_new, v_new):
        _lib.require_device(k_new, v_new)
        for t, name in ((k_new, "k_new"), (v_new, "v_new")):
            _rows_ok(t, name)
            if t.shape[0] != self.BH or t.shape[2] != self.D or t.dtype != self.k.dtype:
                raise ValueError(f"{name} must be [{self.BH}, n, {self.D}] {self.k.dtype}, got "
                                 f"{tuple(t.shape)} {t.dtype}")
        if k_new.shape != v_new.shape or k_new.stride() != v_new.stride():
            raise ValueError("k_new and v_new must share shape and strides")
        n = k_new.shape[1]
        if self.length + n > self.capacity:
            raise ValueError(f"appending {n} tokens to {self.length} exceeds the capacity {self.capacity}")
        return n

    def append(self, k_new, v_new):
        """Append the tokens at original positions length .. length + n - 1
        (k_new, v_new: [BH, n, D] in the cache's dtype); one launch writes them all."""
        n = self._check_new(k_new, v_new)
        with torch.cuda.device(self.device):
            _lib.check(_lib.lib().pa_kv_append(
                _lib.ptr(k_new), _lib.ptr(v_new), k_new.stride(0), k_new.stride(1), _lib.ptr(self.k),
                _lib.ptr(self.v), self.k.stride(0), self.k.stride(1), self.BH, n, self.D, _lib.dtype_code(self.k),
                self.capacity, self.length, self.residue, _lib.stream_of(self.k)), "pa_kv_append")
        self.length += n

    def prepare(self, q, mask, scale=None, qpos0=None, out=None, lse=None, length=None, static_scratch=False,
                k_new=None, v_new=None):
        """A DecodeLaunch of q [BH, nq, D] (nq <= 8, queries at original positions qpos0 ..
        qpos0 + nq - 1, by default the last nq tokens) against the first ``length`` cached
        tokens (default: all).  mask: a polyattn mask object, a MaskSpec or a DeviceMask
        without permutation tables; the cache's basis is applied by the kernel.
        static_scratch: launch pa_decode_fwd_static, which allocates nothing (its split
        partials go to the library's 8 MiB per-GPU scratch; launches that overlap on one
        GPU race).
        k_new, v_new [BH, n, D] (n <= 8): the launch also appends these tokens at positions
        length .. length + n - 1, in the same kernels as the attention (one launch less
        than append() then attend); the cache's length counts them from this call on,
        and every run of the launch writes them again."""
        _lib.require_device(q)
        n_new = 0
        if k_new is not None or v_new is not None:
            if k_new is None or v_new is None:
                raise ValueError("k_new and v_new go together")
            n_new = self._check_new(k_new, v_new)
            if n_new > MAX_QUERIES:
                raise ValueError(f"{n_new} new tokens: one call appends at most {MAX_QUERIES}")
        _rows_ok(q, "q")
        BH, nq, D = q.shape
        if BH != self.BH or D != self.D or q.dtype != self.k.dtype:
            raise ValueError(f"q must be [{self.BH}, nq, {self.D}] {self.k.dtype}")
        if not 1 <= nq <= MAX_QUERIES:
            raise ValueError(f"nq={nq}: decoding takes 1..{MAX_QUERIES} query rows per call")
        new_pos0 = self.length
        total = self.length + n_new
        L = total if length is None else int(length)
        lo = new_pos0 + n_new if n_new else 0   # the appended tokens are attended
        if not lo <= L <= total:
            raise ValueError(f"length={L} outside {lo}..{total}")
        qpos0 = total - nq if qpos0 is None else int(qpos0)
        if qpos0 < 0:
            raise ValueError(f"query positions start at {qpos0} < 0")
        dev = self.device
        dm = mask if isinstance(mask, DeviceMask) else device_mask(mask, self.capacity, dev)
        if dm.perm_q is not None or dm.perm_kv is not None:
            raise ValueError("the mask takes no permutation tables: the cache's basis is applied by the kernel")
        o = out if out is not None else torch.empty_like(q)
        _rows_ok(o, "out")
        if o.shape != q.shape or o.dtype != q.dtype:
            raise ValueError("out must match q in shape and dtype")
        a = _lib.PaDecodeArgs()
        a.q, a.q_sb, a.q_sn, a.nq, a.qpos0 = _lib.ptr(q), q.stride(0), q.stride(1), nq, qpos0
        a.k_cache, a.v_cache = _lib.ptr(self.k), _lib.ptr(self.v)
        a.c_sb, a.c_sn = self.k.stride(0), self.k.stride(1)
        a.capacity, a.length, a.residue_s = self.capacity, L, self.residue
        a.mask = dm.struct()
        a.BH, a.D, a.dtype = BH, D, _lib.dtype_code(q)
        a.scale = float(scale) if scale else float(D ** -0.5)
        a.o, a.o_sb, a.o_sn = _lib.ptr(o), o.stride(0), o.stride(1)
        keep_new = []
        if n_new:
            a.k_new, a.v_new, a.new_sb, a.new_sn = _lib.ptr(k_new), _lib.ptr(v_new), k_new.stride(0), k_new.stride(1)
            a.n_new, a.new_pos0 = n_new, new_pos0
            keep_new = [k_new, v_new]
        if lse is not None:
            _lib.require_device(lse)
            if lse.dtype != torch.float32 or lse.shape != (BH, nq) or lse.stride(1) != 1:
                raise ValueError("lse must be float32 [BH, nq] with unit stride")
            a.lse, a.lse_sb = _lib.ptr(lse), lse.stride(0)
        # the split partials' size is known before any state changes: a static call that
        # would not fit the library's scratch is refused here, not at launch time
        nbytes = ctypes.c_int64(0)
        _lib.check(_lib.lib().pa_decode_workspace(ctypes.byref(a), ctypes.byref(nbytes)), "pa_decode_workspace")
        if static_scratch:
            if nbytes.value > STATIC_SCRATCH_BYTES:
                raise ValueError(f"the split partials need {nbytes.value} bytes, more than the library's "
                                 f"{STATIC_SCRATCH_BYTES}-byte scratch (use static_scratch=False)")
            launch = DecodeLaunch(a, [q, o, lse, dm, self.k, self.v] + keep_new, o, dev, static_scratch=True)
        else:
            ws = torch.empty(max(1, (nbytes.value + 3) // 4), dtype=torch.float32, device=dev)
            a.workspace, a.workspace_bytes = _lib.ptr(ws), ws.numel() * 4
            launch = DecodeLaunch(a, [q, o, lse, dm, ws, self.k, self.v] + keep_new, o, dev)
        self.length = total
        return launch

    def attend(self, q, mask, scale=None, qpos0=None, out=None, lse=None, length=None, static_scratch=False,
               k_new=None, v_new=None):
        """o [BH, nq, D]: see prepare.  If the launch fails, the cache's length is left as it
        was (the appended tokens are not counted)."""
        before = self.length
        launch = self.prepare(q, mask, scale, qpos0, out, lse, length, static_scratch, k_new, v_new)
        try:
            with torch.cuda.device(self.device):
                return launch()
        except Exception:
            self.length = before
            raise
