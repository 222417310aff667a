"""Oracle block index (test infrastructure only).

build_dense: gpu/blockindex.py:32-51 restated on a materialised boolean matrix
(small N).  build: the same result from the streaming C builder (pa_oracle.c),
any N, plus the per-tile wave-group codes.  Both return a dict with kv_idx,
kv_num, kv_partial, elements, live (and wave for the C builder).
"""
import ctypes
import pathlib

import numpy as np

from . import masks

_SO = pathlib.Path(__file__).resolve().parent / "_build" / "libpa_oracle.so"
_LIB = None


class _OTerm(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int32), ("p0", ctypes.c_int32), ("p1", ctypes.c_int32), ("p2", ctypes.c_int32)]


class _OMask(ctypes.Structure):
    _fields_ = [("n_include", ctypes.c_int32), ("n_exclude", ctypes.c_int32), ("terms", _OTerm * 8),
                ("perm_q", ctypes.c_void_p), ("perm_kv", ctypes.c_void_p), ("dense", ctypes.c_void_p),
                ("dense_n", ctypes.c_int64)]


def lib():
    global _LIB
    if _LIB is None:
        if not _SO.exists():
            raise RuntimeError(f"{_SO} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(_SO))
        L.oracle_tile_codes.restype = ctypes.c_int64
        L.oracle_tile_codes.argtypes = [ctypes.POINTER(_OMask), ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_void_p, ctypes.c_int]
        L.oracle_compact.restype = ctypes.c_int32
        L.oracle_compact.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                     ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int64]
        L.oracle_live.restype = ctypes.c_int
        L.oracle_live.argtypes = [ctypes.POINTER(_OMask), ctypes.c_int64, ctypes.c_int64]
        _LIB = L
    return _LIB


def _omask(spec, perm_q, perm_kv, dense, keep):
    include, exclude = spec
    m = _OMask()
    m.n_include, m.n_exclude = len(include), len(exclude)
    for i, t in enumerate(tuple(include) + tuple(exclude)):
        m.terms[i] = _OTerm(*[int(x) for x in t])
    for name, arr in (("perm_q", perm_q), ("perm_kv", perm_kv)):
        if arr is not None:
            a = np.ascontiguousarray(arr, dtype=np.int32)
            keep.append(a)
            setattr(m, name, a.ctypes.data)
    if dense is not None:
        d = np.ascontiguousarray(dense, dtype=np.uint8)
        keep.append(d)
        m.dense, m.dense_n = d.ctypes.data, d.shape[1]
    return m


def tile_codes(spec, N, BQ, A, perm_q=None, perm_kv=None, dense=None, threads=0):
    """(codes uint32 [N/BQ, N/A], live pairs)."""
    assert N % BQ == 0 and N % A == 0
    keep = []
    m = _omask(spec, perm_q, perm_kv, dense, keep)
    codes = np.zeros((N // BQ, N // A), dtype=np.uint32)
    live = lib().oracle_tile_codes(ctypes.byref(m), N, BQ, A, codes.ctypes.data, threads)
    return codes, int(live)


def build(spec, N, BQ, A, perm_q=None, perm_kv=None, dense=None, threads=0):
    """Streaming C restatement of gpu/blockindex.py build (+ wave codes)."""
    codes, live = tile_codes(spec, N, BQ, A, perm_q, perm_kv, dense, threads)
    nq = N // BQ
    kv_num = np.zeros(nq, dtype=np.int32)
    L = lib()
    max_kv = L.oracle_compact(codes.ctypes.data, N, BQ, A, kv_num.ctypes.data, None, None, None, 0)
    kv_idx = np.zeros((nq, max_kv), dtype=np.int32)
    kv_partial = np.zeros((nq, max_kv), dtype=np.int8)
    wave = np.zeros((nq, max_kv), dtype=np.uint32)
    L.oracle_compact(codes.ctypes.data, N, BQ, A, kv_num.ctypes.data, kv_idx.ctypes.data,
                     kv_partial.ctypes.data, wave.ctypes.data, max_kv)
    return dict(kv_idx=kv_idx, kv_num=kv_num, kv_partial=kv_partial, wave=wave,
                elements=int(kv_num.sum()) * BQ * A, live=live, codes=codes)


def build_dense(M, BQ, A):
    """gpu/blockindex.py:32-51 on an explicit boolean matrix M [N, N]."""
    N = M.shape[0]
    assert N % BQ == 0 and N % A == 0
    tiles = M.reshape(N // BQ, BQ, N // A, A)
    any_live = tiles.any(axis=(1, 3))
    all_live = tiles.all(axis=(1, 3))
    counts = any_live.sum(axis=1)
    max_kv = int(counts.max()) if counts.size else 0
    kv_idx = np.zeros((N // BQ, max_kv), dtype=np.int32)
    kv_partial = np.zeros((N // BQ, max_kv), dtype=np.int8)
    for i in range(N // BQ):
        cols = np.flatnonzero(any_live[i])
        kv_idx[i, :cols.size] = cols
        kv_partial[i, :cols.size] = (~all_live[i, cols]).astype(np.int8)
    return dict(kv_idx=kv_idx, kv_num=counts.astype(np.int32), kv_partial=kv_partial,
                elements=int(any_live.sum()) * BQ * A, live=int(M.sum()))


def runs(kv_idx, kv_num):
    """Total count of maximal runs of consecutive kv tiles over all query blocks
    (the 'runs' statistic of gpu/exp8_three_cells.py:46-49)."""
    total = 0
    for i in range(len(kv_num)):
        cols = kv_idx[i, :kv_num[i]]
        if cols.size:
            total += 1 + int((np.diff(cols) > 1).sum())
    return total
