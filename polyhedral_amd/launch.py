"""Launch-configuration sweep table: the call surface of gpu/launchsweep.py.

The HIP kernel's launch shape is set by (BQ, A, D, dtype); the (num_warps,
num_stages) pairs below are the reference's Triton sweep (gpu/launchsweep.py:15-16),
kept so drivers that iterate over them run unchanged.  block_sparse_attention
accepts every pair.
"""
LAUNCH = ((1, 1), (1, 2), (1, 3), (2, 1), (2, 2), (2, 3), (2, 4),
          (4, 1), (4, 2), (4, 3), (8, 2), (8, 3))

_HARD_FLOOR = {"warps": 1, "stages": 1}


def _warn_if_on_boundary(cfg, label=""):
    """A sweep winner on the edge of the sweep means the sweep was too narrow."""
    if not cfg or "None" in cfg:
        return "  <-- NO LAUNCH CONFIG SUCCEEDED"
    w, st = (int(x[1:]) for x in cfg.split("/"))
    ws = sorted({c[0] for c in LAUNCH})
    ss = sorted({c[1] for c in LAUNCH})
    edge = []
    for n, v, lo, hi in (("warps", w, ws[0], ws[-1]), ("stages", st, ss[0], ss[-1])):
        if v == hi:
            edge.append(f"{n} at sweep max")
        elif v == lo and lo > _HARD_FLOOR[n]:
            edge.append(f"{n} at sweep min, floor is {_HARD_FLOOR[n]}")
    return f"  <-- SWEEP TOO NARROW ({'; '.join(edge)}){label}" if edge else ""
