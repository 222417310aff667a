"""pa_decode_fwd_static, the decode entry point that allocates nothing: its split partials
go to the library's per-GPU scratch array instead of a caller workspace.  Through the
C-ABI it gives pa_decode_fwd's output and log-sum-exp bit for bit, on consecutive calls
that share the scratch (the second with a smaller input), and it rejects a call whose
partials exceed the scratch."""
import ctypes

import pytest
import torch

from polyhedral_amd import _lib
from polyhedral_amd import decode as pdec
from polyhedral_amd.registry import numpy_mask
from tests.util import make_qkv

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 8 << 20


def _both(cache, q, name, qpos0, length):
    """(o, lse) from pa_decode_fwd with a workspace and from pa_decode_fwd_static."""
    out = []
    for static in (False, True):
        lse = torch.empty(q.shape[0], q.shape[1], device=q.device)
        launch = cache.prepare(q, numpy_mask(name), qpos0=qpos0, lse=lse, length=length, static_scratch=static)
        assert launch.entry == ("pa_decode_fwd_static" if static else "pa_decode_fwd")
        with torch.cuda.device(q.device):
            o = launch()
        torch.cuda.synchronize()
        out.append((o.clone(), lse.clone()))
    return out


@pytest.mark.parametrize("residue", [0, 16])
def test_static_scratch_equals_workspace_on_consecutive_calls(gpu, residue):
    calls = [  # (heads, capacity, tokens held, nq, length, mask): the second call is smaller
        (8, 4096, 4000, 8, 4000, "band256+lat16"),
        (2, 1024, 700, 3, 650, "sinks4+win256"),
    ]
    for i, (BH, cap, held, nq, L, name) in enumerate(calls):
        print(f"[no-alloc] call {i}: residue={residue} BH={BH} cap={cap} nq={nq} L={L} {name}", flush=True)
        q, k, v = make_qkv(BH, cap, 128, torch.bfloat16, seed=10 * residue + i)
        cache = pdec.KVCache(BH, cap, 128, torch.bfloat16, residue, gpu)
        cache.append(k[:, :held].to(gpu), v[:, :held].to(gpu))
        qd = q[:, L - nq:L].to(gpu)
        (o_w, lse_w), (o_s, lse_s) = _both(cache, qd, name, L - nq, L)
        assert torch.count_nonzero(o_w) > 0
        assert torch.equal(o_s, o_w), f"call {i}: max diff {(o_s.float() - o_w.float()).abs().max().item():.3e}"
        assert torch.equal(lse_s, lse_w)


def test_static_scratch_rejects_oversized_and_workspace_calls(gpu):
    BH, cap = 8, 1024
    q, k, v = make_qkv(BH, cap, 128, torch.bfloat16, seed=5)
    cache = pdec.KVCache(BH, cap, 128, torch.bfloat16, 0, gpu)
    cache.append(k.to(gpu), v.to(gpu))
    launch = cache.prepare(q[:, -8:].to(gpu), numpy_mask("causal"), static_scratch=True)
    need = ctypes.c_int64(0)
    assert _lib.lib().pa_decode_workspace(launch._ref, ctypes.byref(need)) == 0
    assert 0 < need.value <= SCRATCH_BYTES
    launch.args.workspace, launch.args.workspace_bytes = launch.out.data_ptr(), 16
    with pytest.raises(RuntimeError, match="takes no workspace"):
        launch()
    # 4096 heads of one split each: 4096 * 8 * 129 * 4 bytes of partials > 8 MiB
    big = pdec.KVCache(4096, 256, 128, torch.bfloat16, 0, gpu)
    qb = torch.zeros(4096, 8, 128, dtype=torch.bfloat16, device=gpu)
    big.append(qb, qb)
    before = big.length
    with pytest.raises(ValueError, match="scratch"):
        big.attend(qb, numpy_mask("causal"), static_scratch=True)
    assert big.length == before                # refused before the cache's state changed
    # the library refuses it too: the same call prepared with a workspace, sent to the
    # static entry point without one
    launch = big.prepare(qb, numpy_mask("causal"))
    launch.args.workspace, launch.args.workspace_bytes = None, 0
    assert _lib.lib().pa_decode_fwd_static(launch._ref, _lib.stream_of(qb)) == -1
    assert "scratch" in _lib.lib().pa_last_error().decode()
