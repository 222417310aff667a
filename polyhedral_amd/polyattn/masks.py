"""Mask zoo: the predicate families of polyattn (src/polyattn/masks.py:41-290).

Same class names, constructor arguments and interface as the reference
(row_cols(q, N), union_cols(q0, q1, N), live_count(N), dense(N), name, family),
written here as one vectorised predicate per class, ``live(q, kv)``, over numpy
index arrays.  ``terms()`` gives the device predicate the GPU kernels evaluate
(kinds of gpu/masks_gpu.py:9 plus PREFIX_LM).  Combinators the reference
describes but does not implement -- Union, Difference (disjoint peeling,
src/polyattn/experiments/compose.py:7-17) and Permuted (a class-A relabelling,
gpu/test_correctness.py:71) -- are predicates too.

live_count uses per-row closed forms derived here (count of live columns of
row q as a function of q); tests check them against brute force.
"""
import numpy as np

# device predicate kinds (include/polyattn_amd.h); 0..5 = gpu/masks_gpu.py:9
CAUSAL, WINDOW, DILATED, LOCAL_STRIDED, TWOBAND, SINKS, PREFIX_LM, FULL, DENSE = range(9)


class Mask:
    family = "?"
    name = "?"
    data_dependent = False

    def live(self, q, kv):
        """bool array broadcast over integer arrays q, kv (original coordinates)."""
        raise NotImplementedError

    def terms(self):
        """(include, exclude): tuples of (kind, p0, p1, p2) for the device predicate."""
        raise NotImplementedError

    def row_cols(self, q, N):
        return self.live(np.int64(q), np.arange(N, dtype=np.int64))

    def union_cols(self, q0, q1, N):
        out = np.zeros(N, dtype=bool)
        kv = np.arange(N, dtype=np.int64)[None, :]
        for r0 in range(q0, q1, 256):
            rows = np.arange(r0, min(q1, r0 + 256), dtype=np.int64)[:, None]
            out |= self.live(rows, kv).any(axis=0)
        return out

    def _row_counts(self, q, N):
        """live columns of each row in q (int64 array); brute force unless overridden."""
        kv = np.arange(N, dtype=np.int64)[None, :]
        return np.concatenate([self.live(q[i:i + 256, None], kv).sum(axis=1)
                               for i in range(0, len(q), 256)]) if len(q) else np.zeros(0, np.int64)

    def live_count(self, N):
        return int(self._row_counts(np.arange(N, dtype=np.int64), N).sum())

    def dense(self, N):
        i = np.arange(N, dtype=np.int64)
        return self.live(i[:, None], i[None, :])

    def __repr__(self):
        return f"<{type(self).__name__} {self.name}>"


def _clip_len(lo, hi):
    """length of [lo, hi) (arrays), never negative."""
    return np.maximum(0, hi - lo)


class Causal(Mask):
    family, name = "causal", "causal"

    def live(self, q, kv):
        return kv <= q

    def terms(self):
        return ((CAUSAL, 0, 0, 0),), ()

    def _row_counts(self, q, N):
        return np.minimum(q + 1, N)


class SlidingWindow(Mask):
    family = "window"

    def __init__(self, w):
        self.w = w
        self.name = f"window-{w}"

    def live(self, q, kv):
        d = q - kv
        return (d >= 0) & (d < self.w)

    def terms(self):
        return ((WINDOW, self.w, 0, 0),), ()

    def _row_counts(self, q, N):
        return np.minimum(np.minimum(q + 1, N), self.w)


class Dilated(Mask):
    """Causal, live where (q - kv) % s == 0."""
    family = "dilated"

    def __init__(self, s):
        self.s = s
        self.name = f"dilated-{s}"

    def live(self, q, kv):
        d = q - kv
        return (d >= 0) & (d % self.s == 0)

    def terms(self):
        return ((DILATED, self.s, 0, 0),), ()

    def _row_counts(self, q, N):
        return q // self.s + 1  # kv in {q, q - s, ...} >= 0


class SinksWindow(Mask):
    """g absolute sink columns plus a causal window of w."""
    family = "sinks+window"

    def __init__(self, g, w):
        self.g, self.w = g, w
        self.name = f"sinks{g}+win{w}"

    def live(self, q, kv):
        d = q - kv
        return (d >= 0) & ((d < self.w) | (kv < self.g))

    def terms(self):
        return ((SINKS, self.w, self.g, 0),), ()

    def _row_counts(self, q, N):
        sink_hi = np.minimum(self.g, q + 1)                  # sinks: [0, sink_hi)
        win_lo = np.maximum(0, q - self.w + 1)               # window: [win_lo, q + 1)
        return sink_hi + (q + 1 - win_lo) - _clip_len(win_lo, sink_hi)


class PrefixLM(Mask):
    """Bidirectional over the first p positions, causal after."""
    family = "prefix-lm"

    def __init__(self, p):
        self.p = p
        self.name = f"prefixlm-{p}"

    def live(self, q, kv):
        return (kv <= q) | ((q < self.p) & (kv < self.p))

    def terms(self):
        return ((PREFIX_LM, self.p, 0, 0),), ()

    def _row_counts(self, q, N):
        return np.where(q < self.p, min(self.p, N), q + 1)


class LocalStrided(Mask):
    """Causal window w plus every s-th earlier position (d % s == 0)."""
    family = "local+strided"

    def __init__(self, w, s):
        self.w, self.s = w, s
        self.name = f"local{w}+str{s}"

    def live(self, q, kv):
        d = q - kv
        return (d >= 0) & ((d < self.w) | (d % self.s == 0))

    def terms(self):
        return ((LOCAL_STRIDED, self.w, self.s, 0),), ()

    def _row_counts(self, q, N):
        win = np.minimum(q + 1, self.w)
        first_k = -(-self.w // self.s)                       # smallest k with k*s >= w
        return win + np.maximum(0, q // self.s - first_k + 1)


class TwoBand(Mask):
    """Causal offsets d in [0, w1) or [off, off + w2)."""
    family = "two-band"

    def __init__(self, w1, off, w2=None):
        self.w1, self.off, self.w2 = w1, off, w2 or w1
        self.name = f"twoband-{w1}+{off}"

    def live(self, q, kv):
        d = q - kv
        return (d >= 0) & ((d < self.w1) | ((d >= self.off) & (d < self.off + self.w2)))

    def terms(self):
        return ((TWOBAND, self.w1, self.off, self.w2),), ()

    def _row_counts(self, q, N):
        dmax = q + 1                                          # d in [0, q]
        a = np.minimum(self.w1, dmax)
        b_lo, b_hi = self.off, np.minimum(self.off + self.w2, dmax)
        b = _clip_len(b_lo, b_hi)
        return a + b - _clip_len(np.maximum(0, b_lo), np.minimum(a, b_hi))


class Full(Mask):
    family, name = "full", "full"

    def live(self, q, kv):
        return np.ones(np.broadcast(q, kv).shape, dtype=bool)

    def terms(self):
        return ((FULL, 0, 0, 0),), ()


class Union(Mask):
    """live iff any part is live (parts without exclusions)."""
    family = "union"

    def __init__(self, *parts):
        self.parts = parts
        self.name = "|".join(p.name for p in parts)

    def live(self, q, kv):
        out = self.parts[0].live(q, kv)
        for p in self.parts[1:]:
            out = out | p.live(q, kv)
        return out

    def terms(self):
        inc = []
        for p in self.parts:
            i, e = p.terms()
            if e:
                raise ValueError(f"Union part {p.name} has exclusions; not expressible as one predicate")
            inc.extend(i)
        return tuple(inc), ()


class Difference(Mask):
    """live iff `base` is live and `minus` is not: the disjoint peeling of a union."""
    family = "difference"

    def __init__(self, base, minus):
        self.base, self.minus = base, minus
        self.name = f"{base.name}\\{minus.name}"

    def live(self, q, kv):
        return self.base.live(q, kv) & ~self.minus.live(q, kv)

    def terms(self):
        inc, e1 = self.base.terms()
        exc, e2 = self.minus.terms()
        if e1 or e2:
            raise ValueError("nested differences are not expressible as one predicate")
        return inc, exc


class Permuted(Mask):
    """`mask` seen through a class-A relabelling: index-space row r is original perm[r].

    row_cols(r) are the columns c with mask.live(perm[r], perm[c]) -- the matrix
    M[perm][:, perm] that gpu/test_correctness.py:71 materialises."""
    family = "permuted"

    def __init__(self, mask, perm, perm_kv=None):
        self.mask = mask
        self.perm = np.asarray(perm, dtype=np.int64)
        self.perm_kv = self.perm if perm_kv is None else np.asarray(perm_kv, dtype=np.int64)
        self.name = f"perm({mask.name})"

    def live(self, q, kv):
        return self.mask.live(self.perm[q], self.perm_kv[kv])

    def terms(self):
        return self.mask.terms()


class DenseMask(Mask):
    """An explicit boolean matrix in index space (the reference's _Dense wrapper)."""
    family = "dense"

    def __init__(self, M, name="dense"):
        self.M = np.asarray(M, dtype=bool)
        self.name = name

    def live(self, q, kv):
        return self.M[q, kv]

    def row_cols(self, q, N):
        return self.M[q, :N]

    def terms(self):
        return ((DENSE, 0, 0, 0),), ()


def zoo():
    """The masks the reference's test fixture parametrises over (tests/conftest.py:5-7),
    minus the data-dependent document masks, plus the benchmark workloads' families."""
    return [
        Causal(),
        SlidingWindow(128), SlidingWindow(256), SlidingWindow(512), SlidingWindow(1024),
        Dilated(2), Dilated(4), Dilated(8), Dilated(16),
        SinksWindow(4, 256), SinksWindow(4, 1024), SinksWindow(64, 1024),
        LocalStrided(256, 8), LocalStrided(256, 16),
        PrefixLM(1024),
        TwoBand(128, 1024), TwoBand(128, 1000),
    ]
