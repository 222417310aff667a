"""Dense masked attention in torch: the call surface of gpu/reference.py.

attention_reference is the drivers' comparison point (gpu/reference.py:5-13):
fp32 QK^T * scale, -inf where dead, softmax, NaN rows -> 0, @ V, cast to v's dtype.
It runs wherever its tensors are.  The [BH, N, N] score tensor is processed in
row chunks (exact, softmax is per row) so long sequences fit in memory.
"""
import torch


def attention_reference(q, k, v, mask_bool, scale=None, row_chunk=None):
    """q, k, v: [BH, N, D]; mask_bool: [N, N] True where live (or a callable
    (row0, row1) -> bool [row1 - row0, N])."""
    scale = scale or q.shape[-1] ** -0.5
    BH, N, D = q.shape
    if row_chunk is None:
        row_chunk = max(1, min(N, (1 << 28) // max(1, BH * N)))
    kf = k.float()
    vf = v.float()
    out = torch.empty((BH, N, D), dtype=v.dtype, device=q.device)
    for r0 in range(0, N, row_chunk):
        r1 = min(N, r0 + row_chunk)
        m = mask_bool(r0, r1) if callable(mask_bool) else mask_bool[r0:r1]
        s = (q[:, r0:r1].float() @ kf.transpose(-1, -2)) * scale
        s = s.masked_fill(~m.to(s.device)[None], float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
        out[:, r0:r1] = (p @ vf).to(v.dtype)
    return out


def max_abs_err(a, b):
    return (a.float() - b.float()).abs().max().item()
