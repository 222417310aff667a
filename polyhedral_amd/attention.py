"""Block-sparse masked attention forward: the call surface of gpu/triton_attn.py on HIP.

block_sparse_attention keeps the reference signature (gpu/triton_attn.py:185-189),
its defaults, asserts and return value, and runs pa_attn_fwd (a hand-written
gfx950 kernel) instead of the Triton JIT.  Differences a caller can observe:

* SINKS partial tiles apply the sink term on absolute kv (kv < p1), as the ground
  truth gpu/masks_gpu.py:51-52 and gpu/reference.py do; the reference's _live
  drops it (gpu/triton_attn.py:56-59).
* ``kind`` may also be a spec.MaskSpec (unions and set differences of kinds) or a
  spec.DeviceMask (any predicate blockindex.build accepts, explicit matrices
  included), and kind PREFIX_LM = 6 exists.
* num_warps / num_stages are Triton launch knobs; every (num_warps, num_stages) of
  gpu/launchsweep.py:15-16 is accepted and the HIP kernel's shape is fixed by
  (BQ, A, D, dtype), so there is no pipeliner fallback to take.
* gather_mult > 1 (the class-B traffic emulation of gpu/triton_attn.py:108-128)
  runs on the general kernel (the streaming kernel does not emulate it).

Keyword-only extensions: kv_wave_bits (per-wave skip codes; found automatically for
an index made by blockindex.build / to_cuda), kv_bits (element bitmaps of the
partial tiles from blockindex.build_device(bits=True): masking by table lookup,
the predicate is then not evaluated), gather_q / scatter_o (read Q rows
through perm_q and write O rows back to original positions: the class-A
permutation fused into the kernel's loads and stores), lse (write the natural-log
sum-exp per row), prev = (o_prev, lse_prev) (merge a partial over a disjoint
sub-mask by log-sum-exp in the epilogue), out, qblock_order, residue (perm_q and
perm_kv are residue_perm(N, residue): the kernel computes them in closed form),
kv_steps (step descriptors from blockindex.build_steps; found automatically for an
index made by blockindex.build at a streaming tile shape), kernel ("auto": the
streaming kernel whenever its preconditions hold and the index carries its arrays;
"stream": require it; "general": the general kernel).

Two HIP kernels serve the call.  The streaming kernel (f16 / bf16, D = 128, BQ = 128,
A in 16, 32, 64) moves K and V into LDS by DMA and masks from bitmaps; the general
kernel takes every other shape and dtype and can evaluate the predicate itself.
"""
import ctypes

import torch

from . import _lib
from .index import STREAM_TILES, stream_arrays_for, wave_bits_for
from .spec import DeviceMask, MaskSpec, as_perm_tensor

CAUSAL, WINDOW, DILATED, LOCAL_STRIDED, TWOBAND, SINKS, PREFIX_LM = 0, 1, 2, 3, 4, 5, 6

_PIPELINE_FALLBACK = set()


def _assert_kinds_match():
    """The kind constants here and in masks_gpu must agree (gpu/triton_attn.py:32-38)."""
    from . import registry as _m
    mine = dict(CAUSAL=CAUSAL, WINDOW=WINDOW, DILATED=DILATED, LOCAL_STRIDED=LOCAL_STRIDED,
                TWOBAND=TWOBAND, SINKS=SINKS, PREFIX_LM=PREFIX_LM)
    theirs = {k: getattr(_m, k) for k in mine}
    if mine != theirs:
        raise RuntimeError(f"kind constants diverged: triton_attn={mine} masks_gpu={theirs}")


def _rows3(t, name):
    if t.dim() != 3:
        raise ValueError(f"{name} must be [BH, N, D]")
    if t.stride(2) != 1:
        raise ValueError(f"{name} needs a unit-stride last dimension")
    return t


# below this many (batch-head, query block) work-groups the general kernel leaves CUs idle
# (MI355X: 256 CUs), and float32 calls go to the wave-split kernel (one work-group per 16
# query rows)
WSPLIT_MAX_BLOCKS = 256


class Launch:
    """A validated pa_attn_fwd argument block and the tensors its pointers refer to.
    __call__ launches it on the current stream of its device (no re-validation)."""

    def __init__(self, args, keep, out, device, kernel):
        self.args, self.keep, self.out, self.device = args, keep, out, device
        self.kernel = kernel  # "run", "stream", "wsplit" or "general"
        self._ref = ctypes.byref(args)

    def __call__(self):
        _lib.check(_lib.lib().pa_attn_fwd(self._ref, _lib.stream_of(self.out)), "pa_attn_fwd")
        return self.out


def block_sparse_attention(q, k, v, kv_idx, kv_num, kv_partial,
                           kind, p0, p1, p2, BQ, A, scale=None,
                           perm_q=None, perm_kv=None, gather_kv=False,
                           gather_mult=1, gather_scatter=True,
                           num_warps=4, num_stages=2, **ext):
    """q, k, v: [BH, N, D] (float32 / float16 / bfloat16). Returns o [BH, N, D], dtype of q.

    perm_q / perm_kv: int32 [N], permuted position -> ORIGINAL position, used to
    evaluate the mask in original coordinates (identity when None)."""
    launch = prepare(q, k, v, kv_idx, kv_num, kv_partial, kind, p0, p1, p2, BQ, A, scale, perm_q, perm_kv,
                     gather_kv, gather_mult, gather_scatter, num_warps, num_stages, **ext)
    with torch.cuda.device(launch.device):
        return launch()


def prepare(q, k, v, kv_idx, kv_num, kv_partial, kind, p0, p1, p2, BQ, A, scale=None,
            perm_q=None, perm_kv=None, gather_kv=False, gather_mult=1, gather_scatter=True,
            num_warps=4, num_stages=2, *, kv_wave_bits=None, kv_bits=None, gather_q=False, scatter_o=False,
            residue=0, lse=None, prev=None, out=None, qblock_order=None, kv_steps=None, kernel="auto",
            heads_desc=False, wsel=None, run=None):
    """Validate the arguments of block_sparse_attention once and return a Launch.

    heads_desc: issue the heads from the last to the first (the results are the same; a
    pass that follows another over the same tensors then starts where the cache is warm).
    run: a schedule.RunSchedule of this index for these heads (or (schedule, piece)): the
    streaming kernel then runs persistently, a fixed set of work-groups each taking its
    list of (head, query block) items as one stream of steps (same results)."""
    BH, N, D = q.shape
    if perm_kv is None:
        perm_kv = perm_q
    _assert_kinds_match()
    assert N % BQ == 0 and N % A == 0, "cost model and kernel both assume this"
    assert k.shape == v.shape == q.shape
    if int(gather_mult) < 1:
        raise ValueError(f"gather_mult={gather_mult} must be >= 1")
    gather_mult = int(gather_mult)
    _lib.require_device(q, k, v, kv_idx, kv_num, kv_partial)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _rows3(t, n)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share a dtype")
    kv_idx = kv_idx.contiguous()
    kv_num = kv_num.contiguous()
    kv_partial = kv_partial.contiguous()
    nq = N // BQ
    if kv_num.numel() != nq or kv_idx.dim() != 2 or kv_idx.shape[0] != nq or kv_partial.shape != kv_idx.shape:
        raise ValueError(f"block index shapes {tuple(kv_idx.shape)} / {tuple(kv_num.shape)} / "
                         f"{tuple(kv_partial.shape)} do not match N/BQ = {nq}")
    if kv_idx.dtype != torch.int32 or kv_num.dtype != torch.int32 or kv_partial.dtype != torch.int8:
        raise TypeError("block index must be int32 / int32 / int8")
    if kv_wave_bits is None:
        kv_wave_bits = wave_bits_for(kv_idx, BQ, A)
    if kv_wave_bits is not None:
        kv_wave_bits = kv_wave_bits.to(torch.int32).contiguous()
        if kv_wave_bits.shape != kv_idx.shape:
            raise ValueError("kv_wave_bits must have the shape of kv_idx")
    if kernel not in ("auto", "stream", "general", "wsplit"):
        raise ValueError(f"kernel={kernel!r}: expected 'auto', 'stream', 'general' or 'wsplit'")
    # the K / V rows of the step descriptors are in the basis K / V are gathered through
    steps_basis = int(residue) if (gather_kv and residue) else 0
    if kernel not in ("general", "wsplit") and (kv_bits is None or kv_steps is None):
        reg_bits, reg_steps = stream_arrays_for(kv_idx, BQ, A, steps_basis, qblock_order)
        if kv_bits is None and kv_steps is None:
            kv_bits = reg_bits
        if kv_steps is None and (kv_bits is reg_bits or kv_bits is None):
            kv_steps = reg_steps
    if kv_steps is not None and getattr(kv_steps, "order", None) is not qblock_order:
        # the streaming kernel reads its lists in issue order: descriptors laid out for
        # another order are rebuilt for this one from the registered index
        _, kv_steps = stream_arrays_for(kv_idx, BQ, A, steps_basis, qblock_order)
        if kv_steps is None:
            raise ValueError("kv_steps were laid out for another qblock_order (build them with "
                             "build_steps(..., order=qblock_order))")
    if kv_steps is not None and getattr(kv_steps, "residue_s", steps_basis) != steps_basis:
        raise ValueError(f"kv_steps hold K/V rows in the residue-{kv_steps.residue_s} basis; this call gathers "
                         f"in the residue-{steps_basis} basis (build them with build_steps(..., residue))")

    dev = q.device
    if isinstance(kind, DeviceMask):
        if perm_q is not None:
            raise ValueError("a DeviceMask carries its own permutation; pass no perm_q / perm_kv")
        dmask = kind
    else:
        dmask = DeviceMask(MaskSpec.of(kind, p0, p1, p2), as_perm_tensor(perm_q, dev),
                           as_perm_tensor(perm_kv, dev))
    o = out if out is not None else torch.empty_like(q)
    _rows3(o, "out")
    if o.shape != q.shape or o.dtype != q.dtype:
        raise ValueError("out must match q in shape and dtype")

    args = _lib.PaAttnArgs()
    args.q, args.k, args.v, args.o = _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o)
    args.q_sb, args.q_sn = q.stride(0), q.stride(1)
    args.k_sb, args.k_sn = k.stride(0), k.stride(1)
    args.v_sb, args.v_sn = v.stride(0), v.stride(1)
    args.o_sb, args.o_sn = o.stride(0), o.stride(1)
    args.BH, args.N, args.D = BH, N, D
    args.dtype = _lib.dtype_code(q)
    args.scale = float(scale or D ** -0.5)
    args.BQ, args.A = BQ, A
    args.kv_idx, args.kv_num, args.kv_partial = _lib.ptr(kv_idx), _lib.ptr(kv_num), _lib.ptr(kv_partial)
    args.kv_wave_bits = _lib.ptr(kv_wave_bits)
    args.pitch = kv_idx.shape[1]
    if kv_bits is not None:
        bits_off, bits_pool = kv_bits
        _lib.require_device(bits_off, bits_pool)
        if bits_off.shape != kv_idx.shape or bits_off.dtype != torch.int32 or bits_pool.dtype != torch.int32:
            raise ValueError("kv_bits must be (int32 offsets shaped like kv_idx, int32 bitmap pool)")
        args.kv_bits_off, args.kv_bits = _lib.ptr(bits_off), _lib.ptr(bits_pool)
    args.mask = dmask.struct()
    gathers_kv = bool(gather_kv) and (perm_kv is not None or bool(residue))
    args.gather_q, args.gather_kv, args.scatter_o = int(bool(gather_q)), int(gathers_kv), int(bool(scatter_o))
    if residue:
        # perm_q = perm_kv = residue_perm(N, residue), evaluated in closed form by the kernel
        qn = N // residue
        if N % residue or qn & (qn - 1):
            raise ValueError(f"closed-form residue basis needs N/s a power of two (N={N}, s={residue})")
        args.residue_s, args.residue_qlog2 = int(residue), qn.bit_length() - 1
    if lse is not None:
        _lib.require_device(lse)
        if lse.dtype != torch.float32 or lse.shape != (BH, N) or lse.stride(1) != 1:
            raise ValueError("lse must be float32 [BH, N] with unit row stride")
        args.lse, args.lse_sb = _lib.ptr(lse), lse.stride(0)
    if prev is not None:
        o_prev, lse_prev = prev
        _lib.require_device(o_prev, lse_prev)
        _rows3(o_prev, "prev o")
        if o_prev.shape != q.shape or lse_prev.shape != (BH, N) or lse_prev.dtype != torch.float32:
            raise ValueError("prev must be (o [BH, N, D], lse float32 [BH, N])")
        if lse is not None and lse.stride(0) != lse_prev.stride(0):
            raise ValueError("lse and prev lse must share their row stride")
        if lse_prev.stride(1) != 1:
            raise ValueError("prev lse needs a unit row stride")
        args.prev_o, args.prev_dtype = _lib.ptr(o_prev), _lib.dtype_code(o_prev)
        args.prev_sb, args.prev_sn = o_prev.stride(0), o_prev.stride(1)
        args.prev_lse = _lib.ptr(lse_prev)
        args.lse_sb = lse_prev.stride(0)
    if qblock_order is not None:
        qblock_order = qblock_order.to(device=dev, dtype=torch.int32).contiguous()
        if qblock_order.numel() != nq:
            raise ValueError("qblock_order must have N/BQ entries")
        args.qblock_order = _lib.ptr(qblock_order)
    # the streaming kernel's preconditions (pa_attn_fwd rejects kv_steps otherwise)
    pitch = kv_idx.shape[1]
    why = None
    if gather_mult > 1:
        why = "gather_mult > 1 (the class-B traffic emulation runs on the general kernel)"
    elif q.dtype not in (torch.float16, torch.bfloat16) or D != 128 or (BQ, A) not in STREAM_TILES:
        why = f"dtype {q.dtype}, D={D}, tile {BQ}x{A} (needs f16/bf16, D=128, BQ=128, A in 16/32/64)"
    elif gathers_kv and not residue:
        why = "K/V gathered through a permutation table (only the closed-form residue basis)"
    elif pitch and kv_bits is None:
        why = "no partial-tile bitmaps for this index"
    elif pitch and kv_steps is None:
        why = "no step descriptors for this index"
    if kernel == "stream" and why is not None:
        raise ValueError(f"the streaming kernel cannot take this call: {why}")
    use_stream = kernel not in ("general", "wsplit") and why is None and pitch > 0
    if use_stream:
        _lib.require_device(kv_steps)
        if kv_steps.dtype != torch.int32 or kv_steps.dim() != 3 or kv_steps.shape[0] != nq \
                or kv_steps.shape[2] != 16 or not kv_steps.is_contiguous():
            raise ValueError("kv_steps must be contiguous int32 [N/BQ, steps, 16]")
        args.kv_steps, args.steps_pitch = _lib.ptr(kv_steps), kv_steps.shape[1]
    use_run = use_stream and run is not None
    if use_run:
        # run = (schedule, the piece of its rows this call is)
        run, piece = run if isinstance(run, tuple) else (run, 0)
        if (run.BH, run.N, run.residues[piece]) != (BH, N, steps_basis):
            raise ValueError(f"run schedule built for BH={run.BH}, N={run.N}, residue {run.residues[piece]}; "
                             f"this call has BH={BH}, N={N}, residue {steps_basis}")
        for t, n in ((k, "k"), (v, "v")):
            if t.stride(0) != N * t.stride(1):
                raise ValueError(f"the persistent kernel needs {n} with batch stride N * row stride")
        args.run_steps, args.run_start, args.run_groups = _lib.ptr(run.run), _lib.ptr(run.start), run.groups
    # the wave-split kernel (pa_attn_args.wave_split): float32 grids of fewer query blocks
    # than the chip has CUs, where one work-group per block would leave most of it idle
    why_ws = None
    if q.dtype != torch.float32 or D not in (64, 128) or BQ % 32 or A % 32:
        why_ws = f"dtype {q.dtype}, D={D}, tile {BQ}x{A} (needs float32, D = 64 or 128, BQ and A multiples of 32)"
    elif kv_wave_bits is None and kv_idx.shape[1] > 0:
        why_ws = "no wave-group codes for this index"
    elif (dmask.perm_q is not None or dmask.perm_kv is not None or gather_q or gathers_kv or scatter_o
          or residue):
        why_ws = "a permutation"
    elif gather_mult > 1 or prev is not None:
        why_ws = "class-B emulation or a merge input"
    if kernel == "wsplit" and why_ws is not None:
        raise ValueError(f"the wave-split kernel cannot take this call: {why_ws}")
    use_ws = (not use_stream and why_ws is None and
              (kernel == "wsplit" or (kernel == "auto" and BH * nq < WSPLIT_MAX_BLOCKS)))
    args.wave_split = 1 if use_ws else 0
    args.heads_desc = 1 if heads_desc else 0
    wsel_t = None
    if gather_mult > 1:
        # [1, 0, ...] per batch-head, as gpu/triton_attn.py:202-205: runtime weights keep the
        # extra K reads alive and leave the result unchanged (wsel= overrides them)
        if wsel is None:
            wsel_t = torch.zeros(BH, gather_mult, dtype=q.dtype, device=dev)
            wsel_t[:, 0] = 1
        else:
            wsel_t = wsel.to(device=dev, dtype=q.dtype).contiguous()
            if wsel_t.shape != (BH, gather_mult):
                raise ValueError(f"wsel must be [BH, gather_mult] = [{BH}, {gather_mult}]")
        args.gather_mult, args.gather_scatter = gather_mult, 1 if gather_scatter else 0
        args.wsel, args.wsel_sb = _lib.ptr(wsel_t), wsel_t.stride(0)
    keep = [q, k, v, o, kv_idx, kv_num, kv_partial, kv_wave_bits, kv_bits, dmask, lse, prev, qblock_order,
            kv_steps, wsel_t, run]
    return Launch(args, keep, o, dev,
                  "run" if use_run else "stream" if use_stream else "wsplit" if use_ws else "general")
