"""Shared helpers for the tests: seeded inputs, tolerances, oracle references."""
import numpy as np
import torch

# tolerances of the path against the float64 oracle: fp32 1e-5 absolute; bf16 max-abs
# 2e-2 and mean-abs 2e-3; fp16 the reference gate's 3e-3 (gpu/test_correctness.py:23)
TOL = {torch.float32: (1e-5, None), torch.bfloat16: (2e-2, 2e-3), torch.float16: (3e-3, None)}

TILES_GATE = [(128, 128), (128, 32), (64, 64), (32, 32), (16, 16), (128, 16), (16, 128)]


def make_qkv(BH, N, D, dtype, seed=0, k_scale_first=None):
    """CPU torch.Generator(seed): q, k, v drawn in that order as fp32 randn, then cast."""
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(BH, N, D, generator=g) for _ in range(3))
    if k_scale_first is not None:
        n, f = k_scale_first
        k[:, :n] *= f
    return tuple(x.to(dtype) for x in (q, k, v))


def as64(x):
    return x.detach().float().cpu().numpy().astype(np.float64)


def check_close(out, want, dtype, what=""):
    """out: device tensor; want: float64 array.  Returns (max, mean) abs error."""
    err = np.abs(as64(out) - want)
    mx, mean = float(err.max()), float(err.mean())
    tmax, tmean = TOL[dtype]
    assert mx <= tmax, f"{what}: max abs err {mx:.3e} > {tmax:g}"
    if tmean is not None:
        assert mean <= tmean, f"{what}: mean abs err {mean:.3e} > {tmean:g}"
    return mx, mean
