"""GPU block-index builder: the call surface of gpu/blockindex.py (BlockIndex, build, to_cuda).

build(mask, N, BQ, A) gives the same BlockIndex as gpu/blockindex.py:32-51 --
ascending live KV tiles per query block, zero padded to max_kv columns, int32 /
int32 / int8, elements = listed tiles * BQ * A, live = live pairs -- but the
predicate is evaluated and tiled on the GPU (pa_index_classify / pa_index_compact)
instead of materialising the N x N mask on the host.  The device arrays stay
cached on the BlockIndex, so to_cuda hands them out without a second upload; the
numpy fields are filled from one device-to-host copy to keep the reference's
dataclass contract.

Extensions (keyword-only): ``perm`` / ``perm_kv`` build the index of a class-A
relabelled mask without materialising M[perm][:, perm]; ``kv_wave_bits`` is the
per-tile code of 2 bits per 32-row x 32-column wave group (some live / all live),
which the attention kernel uses to skip or mask at wave granularity.  For the tile
shapes the streaming attention kernel takes (STREAM_TILES), build() also makes the
partial-tile bitmaps (pa_index_bits) and the step descriptors (pa_index_steps) and
keeps them with the index, so block_sparse_attention finds them from kv_idx alone.
"""
import ctypes
import weakref
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import _lib
from .spec import device_mask

# (BQ, A) tile shapes of the streaming attention kernel (f16 / bf16, D = 128)
STREAM_TILES = ((128, 16), (128, 32), (128, 64))

# id(kv_idx device tensor) -> (weakref to it, dict of the arrays made with it: wave
# codes, bitmaps, step descriptors, and its BQ, A), so the reference call surface
# (which passes only kv_idx / kv_num / kv_partial) still gets per-wave skipping and
# the streaming kernel.  Keyed by id because tensors compare elementwise.
_EXTRAS = {}


def _register(kv_idx, BQ, A, **arrays):
    key = id(kv_idx)
    entry = _EXTRAS.get(key)
    if entry is None or entry[0]() is not kv_idx:
        entry = (weakref.ref(kv_idx), dict(BQ=BQ, A=A, steps={}))
        _EXTRAS[key] = entry
        weakref.finalize(kv_idx, _EXTRAS.pop, key, None)
    steps = arrays.pop("steps", None)
    if steps:
        entry[1]["steps"].update(steps)
    entry[1].update(arrays)


def _extras(kv_idx, BQ, A):
    entry = _EXTRAS.get(id(kv_idx))
    if entry is None or entry[0]() is not kv_idx or (entry[1]["BQ"], entry[1]["A"]) != (BQ, A):
        return {}
    return entry[1]


def build_steps(kv_idx, kv_num, kv_partial, wave, bits_off, N, BQ, A, residue=0, order=None):
    """Step descriptors [N/BQ, ceil(pitch * A / 64), 16] int32 (pa_index_steps) whose
    K / V rows are in the residue-s basis (residue > 0, N / s a power of two) or in index
    space (residue = 0); None for an index whose every list is empty.  The lists are laid
    out in the issue order ``order`` (int32 [N/BQ] device tensor, the qblock_order of the
    launches that use them; None: index order).  The tensor carries the basis and the order
    as attributes ``residue_s`` and ``order``."""
    nq, pitch = kv_idx.shape
    sp = (pitch * A + 63) // 64
    if sp == 0:
        return None
    qlog2 = 0
    if residue:
        qn = N // residue
        if N % residue or qn & (qn - 1):
            raise ValueError(f"closed-form residue basis needs N/s a power of two (N={N}, s={residue})")
        qlog2 = qn.bit_length() - 1
    steps = torch.empty((nq, sp, 16), dtype=torch.int32, device=kv_idx.device)
    with torch.cuda.device(kv_idx.device):
        _lib.check(_lib.lib().pa_index_steps(_lib.ptr(kv_idx), _lib.ptr(kv_num), _lib.ptr(kv_partial),
                                             _lib.ptr(wave), _lib.ptr(bits_off), pitch, N, BQ, A, int(residue),
                                             qlog2, _lib.ptr(order), _lib.ptr(steps), sp, _lib.stream_of(steps)),
                   "pa_index_steps")
    steps.residue_s = int(residue)
    steps.order = order
    return steps


@dataclass
class BlockIndex:
    BQ: int
    A: int
    N: int
    kv_idx: np.ndarray       # [n_q_blocks, max_kv] int32: kv tile ids, ascending
    kv_num: np.ndarray       # [n_q_blocks] int32
    kv_partial: np.ndarray   # [n_q_blocks, max_kv] int8: 1 if the mask must be applied
    elements: int            # listed tiles * BQ * A
    live: int                # live (q, kv) pairs
    kv_wave_bits: Optional[np.ndarray] = None  # [n_q_blocks, max_kv] uint32 wave-group codes
    _device: Optional[tuple] = field(default=None, repr=False, compare=False)

    @property
    def waste(self):
        return self.elements / self.live

    @property
    def tiles(self):
        return self.elements // (self.BQ * self.A)

    @property
    def max_kv(self):
        return int(self.kv_idx.shape[1])


def _default_device(device):
    if device is None:
        device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else None
    if device is None or torch.device(device).type != "cuda":
        raise RuntimeError("blockindex.build runs on the GPU only (no host builder in the product path)")
    return torch.device(device)


def build_device(mask, N, BQ, A, *, perm=None, perm_kv=None, device=None, bits=False, steps=False,
                 residue=0):
    """Build on the GPU; returns (kv_idx, kv_num, kv_partial, kv_wave_bits, tiles, live) with
    device tensors and host ints.  One synchronisation (to size the padded lists).

    bits=True appends (kv_bits_off, kv_bits): element bitmaps of the partial tiles
    (pa_index_bits), so the attention kernel masks by table lookup.  steps=True (which
    implies bits) appends the step descriptors of the streaming kernel (None when every
    list is empty), with K / V rows in the residue-``residue`` basis (0: index space)."""
    bits = bits or steps
    assert N % BQ == 0 and N % A == 0
    dev = _default_device(device)
    dm = device_mask(mask, N, dev, perm=perm, perm_kv=perm_kv)
    nq, nk = N // BQ, N // A
    codes = torch.empty(nq * nk, dtype=torch.int32, device=dev)
    kv_num = torch.empty(nq, dtype=torch.int32, device=dev)
    totals = torch.empty(3, dtype=torch.int64, device=dev)
    L = _lib.lib()
    ms = dm.struct()
    with torch.cuda.device(dev):
        stream = _lib.stream_of(codes)
        _lib.check(L.pa_index_classify(ctypes.byref(ms), N, BQ, A, _lib.ptr(codes), _lib.ptr(kv_num), _lib.ptr(totals),
                                       stream), "pa_index_classify")
        tiles, live, max_kv = (int(x) for x in totals.cpu())
        kv_idx = torch.empty((nq, max_kv), dtype=torch.int32, device=dev)
        kv_partial = torch.empty((nq, max_kv), dtype=torch.int8, device=dev)
        wave = torch.empty((nq, max_kv), dtype=torch.int32, device=dev)
        _lib.check(L.pa_index_compact(_lib.ptr(codes), _lib.ptr(kv_num), N, BQ, A, _lib.ptr(kv_idx),
                                      _lib.ptr(kv_partial), _lib.ptr(wave), max_kv, stream),
                   "pa_index_compact")
        out = (kv_idx, kv_num, kv_partial, wave, tiles, live)
        if bits:
            part = kv_partial.to(torch.int64).sum(1)
            part_base = torch.cumsum(part, 0) - part
            n_part = int(part.sum())
            wpr = (A + 31) // 32
            pool = torch.zeros(max(1, n_part * BQ * wpr), dtype=torch.int32, device=dev)
            off = torch.full((nq, max_kv), -1, dtype=torch.int32, device=dev)
            _lib.check(L.pa_index_bits(ctypes.byref(ms), N, BQ, A, _lib.ptr(kv_idx), _lib.ptr(kv_num),
                                       _lib.ptr(kv_partial), max_kv, _lib.ptr(part_base), _lib.ptr(off),
                                       _lib.ptr(pool), stream), "pa_index_bits")
            out = out + ((off, pool),)
            _register(kv_idx, BQ, A, bits=(off, pool), N=N, arrays=(kv_num, kv_partial, wave))
        if steps:
            st = build_steps(kv_idx, kv_num, kv_partial, wave, out[6][0], N, BQ, A, residue)
            out = out + (st,)
            _register(kv_idx, BQ, A, steps={int(residue): st}, N=N, arrays=(kv_num, kv_partial, wave))
    _register(kv_idx, BQ, A, wave=wave)
    return out


def build(mask, N, BQ, A, *, perm=None, perm_kv=None, device=None):
    """gpu/blockindex.py:32 build(mask, N, BQ, A), computed on the GPU."""
    stream = (BQ, A) in STREAM_TILES
    kv_idx, kv_num, kv_partial, wave, tiles, live = build_device(mask, N, BQ, A, perm=perm, perm_kv=perm_kv,
                                                                 device=device, steps=stream)[:6]
    return BlockIndex(BQ, A, N, kv_idx.cpu().numpy(), kv_num.cpu().numpy(), kv_partial.cpu().numpy(),
                      tiles * BQ * A, live, wave.cpu().numpy().view(np.uint32),
                      _device=(kv_idx, kv_num, kv_partial, wave))


def to_cuda(bi, device="cuda"):
    """gpu/blockindex.py:54-58: (kv_idx, kv_num, kv_partial) on the device."""
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    if bi._device is not None and bi._device[0].device == dev:
        return bi._device[:3]
    kv_idx = torch.from_numpy(np.ascontiguousarray(bi.kv_idx)).to(dev)
    out = (kv_idx, torch.from_numpy(np.ascontiguousarray(bi.kv_num)).to(dev),
           torch.from_numpy(np.ascontiguousarray(bi.kv_partial)).to(dev))
    if bi.kv_wave_bits is not None and dev.type == "cuda":
        wave = torch.from_numpy(np.ascontiguousarray(bi.kv_wave_bits).view(np.int32)).to(dev)
        _register(kv_idx, bi.BQ, bi.A, wave=wave)
    return out


def wave_bits_for(kv_idx, BQ, A):
    """The wave-group codes registered for this kv_idx tensor at this tile shape, or None."""
    wave = _extras(kv_idx, BQ, A).get("wave")
    return wave if wave is not None and wave.shape == kv_idx.shape else None


def stream_arrays_for(kv_idx, BQ, A, residue=0, order=None):
    """(bitmaps, step descriptors in the residue basis and the issue order ``order``)
    registered for this kv_idx tensor, building the descriptors for a new basis or order
    from the registered index arrays; (None, None) when the index was not built with
    bitmaps."""
    ex = _extras(kv_idx, BQ, A)
    bits = ex.get("bits")
    if bits is None:
        return None, None
    if order is None:
        steps = ex["steps"].get(int(residue))
    else:
        hit = ex.setdefault("ordered", {}).get((int(residue), id(order)))
        steps = hit[1] if hit is not None and hit[0] is order else None
    if steps is None and "arrays" in ex:
        kv_num, kv_partial, wave = ex["arrays"]
        steps = build_steps(kv_idx, kv_num, kv_partial, wave, bits[0], ex["N"], BQ, A, residue, order)
        if order is None:
            ex["steps"][int(residue)] = steps
        else:
            ex["ordered"][(int(residue), id(order))] = (order, steps)
    return bits, steps
