#!/usr/bin/env python3
"""Benchmark of the block-sparse masked attention forward on one MI355X.

Default: the L=16384, H=32, D=128 bf16 workload (band-256 | lattice-16, split into
band-256 in the identity basis and lattice-16 minus band in the rp16 basis, merged
by log-sum-exp), inputs resident in HBM, one step = one forward over the batch;
then the other four workloads (and the dilated one in both bases) as a per-workload
block of the same line.  Prints ONE JSON line on stdout (the driver's contract);
progress goes to stderr.

  python bench.py [--steps K] [--warmup W] [--workload NAME] [--no-cpu] [--no-configs]
  python bench.py --all [--report PATH]    every workload and variant, with every extra

Each workload first runs forwards back to back for --settle-ms of wall time (the
GPU's clocks rise over the first ~100 ms of load), then W untimed steps, then K
timed back-to-back steps between two device synchronisations.  HIP events around
each kernel launch, on the launch stream, give the per-launch durations the roofline
uses: live FLOPs of the launch and its algorithmic bytes over its duration, against
the dense MFMA peak and 8 TB/s; the bound is the one the arithmetic intensity picks.
After the timed region, the CPU leg times the oracle (gpu/reference.py restated:
dense masked fp32 attention, torch on the host's cores) on a bounded sample of the
same workload and checks the timed output against the oracle's float64 attention on
sampled rows of every head (`parity`).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "block-sparse attn fwd ms + live-FLOP TFLOP/s (% bf16 MFMA peak), L=16k H=32 D=128"
PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}   # dense MFMA, MI355X
HBM_GBPS = 8000.0
# oracle predicate name of each workload's whole mask
ORACLE_NAME = {"window128-L1k": "window-128", "dilated8-L8k": "dilated-8", "bandlat-L16k": "band256+lat16",
               "sinkwin-L32k": "sinks64+win1024", "prefixlat-L64k": "prefixlm-2048",
          "bandlat32-L64k": "band256+lat32"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _dt(dtype):
    import torch
    return {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}[dtype]


def measure(plan_launches, steps, warmup, every=4):
    """(wall ms per step, per-launch mean ms) over `steps` back-to-back forwards.  HIP
    events bracket each launch of every `every`-th step (all steps when there are fewer
    than 2 * every): an event record costs a few microseconds of wall time, so the other
    steps run without them."""
    import torch
    for _ in range(warmup):
        for launch in plan_launches:
            launch()
    torch.cuda.synchronize()
    n = len(plan_launches)
    every = every if steps >= 2 * every else 1
    timed = range(0, steps, every)
    evs = {s: [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)] for s in timed}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        e = evs.get(s)
        if e is None:
            for launch in plan_launches:
                launch()
            continue
        e[0].record()
        for i, launch in enumerate(plan_launches):
            launch()
            e[i + 1].record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    per = [sum(evs[s][i].elapsed_time(evs[s][i + 1]) for s in timed) / len(timed) for i in range(n)]
    return wall_ms, per


def measure_isolated(plan_launches, reps, flush_mib=512):
    """The reference's timing protocol (gpu/bench.py:11-24), with the flush sized for this
    GPU: before each forward a flush_mib MiB buffer is zeroed (more than the 256 MiB
    memory-side cache), then one forward is timed alone with events and the device is
    synchronised.  Returns the median in ms."""
    import statistics

    import torch
    dev = plan_launches[0].device
    cache = torch.empty(flush_mib * (1 << 20) // 4, dtype=torch.int32, device=dev)
    out = []
    for _ in range(reps):
        cache.zero_()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for launch in plan_launches:
            launch()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e))
    del cache
    return statistics.median(out)


def measure_graph(plan_launches, steps_per_graph=10, rounds=3, min_ms=50.0):
    """The device's rate for a forward: `steps_per_graph` forwards captured in one HIP
    graph and replayed back to back (a forward of a few microseconds is otherwise paced
    by the host's launches).  Median over `rounds` rounds of replays, each at least
    `min_ms` long.  Returns ms per forward."""
    import torch
    dev = plan_launches[0].device
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for _ in range(steps_per_graph):
                for launch in plan_launches:
                    launch()
    torch.cuda.current_stream(dev).wait_stream(side)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    per = max(1e-3, (time.perf_counter() - t0) * 1e3)
    reps = max(1, int(min_ms / per))
    out = []
    for _ in range(rounds):
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(reps):
            g.replay()
        ev[1].record()
        torch.cuda.synchronize()
        out.append(ev[0].elapsed_time(ev[1]) / (reps * steps_per_graph))
    del g
    return sorted(out)[len(out) // 2]


def measure_permute(q, k, v, s, reps=50, warmup=10):
    """The class-A relabelling as standalone HBM gather / scatter kernels (the path of
    gpu/permute.py:22-24 and gpu/exp5_amortisation.py, which the fused attention path does
    not need): Q, K, V gathered through the residue-s permutation by one pa_permute_stack
    launch, and O scattered back by pa_permute_rows.  Algorithmic bytes: each tensor
    read once and written once."""
    import torch

    from polyhedral_amd import perm as pperm
    N = q.shape[1]
    p = pperm.residue_perm_device(N, s, q.device)
    o = torch.empty_like(q)
    ob = torch.empty_like(q)

    def timed(fn):
        for _ in range(warmup):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(reps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / reps

    ms_g = timed(lambda: pperm.permute_stack([q, k, v], p, with_positions=True))
    ms_s = timed(lambda: pperm.permute_rows(o, p, inverse=True, out=ob))
    tb = q.numel() * q.element_size()

    def entry(ms, nbytes):
        gbs = nbytes / (ms * 1e-3) / 1e9
        return dict(ms=round(ms, 5), bytes=nbytes, gb_per_s=round(gbs, 1),
                    roofline=dict(bound="hbm", achieved=round(gbs, 1), peak=HBM_GBPS, unit="GB/s",
                                  frac=round(gbs / HBM_GBPS, 4)))
    return dict(residue=s, gather_qkv=entry(ms_g, 3 * 2 * tb), scatter_o=entry(ms_s, 2 * tb),
                note="algorithmic bytes = 2 x tensor bytes per tensor moved; gather_qkv is one "
                     "pa_permute_stack launch (Q, K, V and the position ids), scatter_o one pa_permute_rows")


def measure_decode(wl, q, k, v, residues=(0, 16), reps=200, warmup=20):
    """One decode step of the workload's mask against a cache of all L tokens: the newest
    token's K / V appended and its query row attended to the cache, in one pa_decode_fwd
    call (split kernel + merge; the split's work-group owning the new row writes it,
    rewriting the same row every step), captured in a HIP graph and replayed (the step is
    a few microseconds of kernels; ~150 ms of replays settle the clocks, then the median
    of 3 rounds).  The same step as pa_kv_append then pa_decode_fwd is
    timed beside it (`separate_ms_per_token`), and both are also timed launched eagerly and
    as a graph of ten steps (`graph10_ms_per_token`: the device's rate, where a one-step
    replay is bound by the host's graph launch).
    Algorithmic bytes: the live keys' K and V rows, the appended rows, q and o."""
    import ctypes

    import torch

    from polyhedral_amd import _lib
    from polyhedral_amd import decode as pdec
    H, L, D = wl.H, wl.L, wl.D
    live = int(np.asarray(wl.union.row_cols(L - 1, L), dtype=bool).sum())
    rb = D * q.element_size()
    nbytes = H * (2 * live * rb + 2 * rb + 2 * rb)
    out = {}
    for s in residues:
        kn, vn, qn = k[:, L - 1:].contiguous(), v[:, L - 1:].contiguous(), q[:, L - 1:].contiguous()
        # the step as one call (append inside the decode kernels) ...
        cache = pdec.KVCache(H, L, D, q.dtype, s, q.device)
        cache.append(k[:, :L - 1], v[:, :L - 1])
        fused = cache.prepare(qn, wl.union, k_new=kn, v_new=vn)
        # ... and as pa_kv_append followed by the decode call, on a second cache
        cache2 = pdec.KVCache(H, L, D, q.dtype, s, q.device)
        cache2.append(k[:, :L - 1], v[:, :L - 1])
        cache2.append(kn, vn)
        attend = cache2.prepare(qn, wl.union)
        lib = _lib.lib()
        app_args = (_lib.ptr(kn), _lib.ptr(vn), kn.stride(0), kn.stride(1), _lib.ptr(cache2.k), _lib.ptr(cache2.v),
                    cache2.k.stride(0), cache2.k.stride(1), H, 1, D, _lib.dtype_code(kn), L, L - 1, cache2.residue)

        def separate():
            _lib.check(lib.pa_kv_append(*app_args, _lib.stream_of(kn)), "pa_kv_append")
            attend()

        def timed(step, out_t):
            step()
            torch.cuda.synchronize()
            eager_out = out_t.clone()
            g = torch.cuda.CUDAGraph()
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                with torch.cuda.graph(g, stream=side):
                    step()
            torch.cuda.current_stream().wait_stream(side)
            # clocks settle under ~150 ms of replays (a step is tens of microseconds, and the
            # GPU may have idled since the forward's timing), then 3 rounds, the median
            t_end = time.perf_counter() + 0.15
            while time.perf_counter() < t_end:
                for _ in range(warmup):
                    g.replay()
                torch.cuda.synchronize()
            same = torch.equal(out_t, eager_out)
            rounds = []
            for _ in range(3):
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                ev[0].record()
                for _ in range(reps):
                    g.replay()
                ev[1].record()
                torch.cuda.synchronize()
                rounds.append(ev[0].elapsed_time(ev[1]) / reps)
            ms = sorted(rounds)[1]
            # ten steps in one graph: a one-step replay of a step this short can be bound by
            # the host's graph launch, so this is the rate the device sustains
            g10 = torch.cuda.CUDAGraph()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                with torch.cuda.graph(g10, stream=side):
                    for _ in range(10):
                        step()
            torch.cuda.current_stream().wait_stream(side)
            for _ in range(5):
                g10.replay()
            torch.cuda.synchronize()
            same = same and torch.equal(out_t, eager_out)
            rounds10 = []
            for _ in range(3):
                ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
                ev[0].record()
                for _ in range(reps // 10):
                    g10.replay()
                ev[1].record()
                torch.cuda.synchronize()
                rounds10.append(ev[0].elapsed_time(ev[1]) / (reps // 10 * 10))
            ms10 = sorted(rounds10)[1]
            # eager steps for comparison (host launch overhead included)
            t0 = time.perf_counter()
            for _ in range(50):
                step()
            torch.cuda.synchronize()
            return ms, (time.perf_counter() - t0) * 1e3 / 50, same, ms10

        ms, eager_ms, same, ms10 = timed(fused, fused.out)
        sep_ms, sep_eager_ms, _, sep_ms10 = timed(separate, attend.out)
        agree = torch.equal(fused.out, attend.out)
        gbs = nbytes / (ms * 1e-3) / 1e9
        gbs10 = nbytes / (ms10 * 1e-3) / 1e9
        out["identity" if s <= 1 else f"rp{s}"] = dict(
            ms_per_token=round(ms, 5), eager_ms_per_token=round(eager_ms, 5), tokens_per_s=round(1e3 / ms, 1),
            graph10_ms_per_token=round(ms10, 5),
            separate_ms_per_token=round(sep_ms, 5), separate_eager_ms_per_token=round(sep_eager_ms, 5),
            separate_graph10_ms_per_token=round(sep_ms10, 5),
            graph_equals_eager=same, one_call_equals_separate=agree, bytes=nbytes, gb_per_s=round(gbs, 1),
            roofline=dict(bound="hbm", achieved=round(gbs10, 1), peak=HBM_GBPS, unit="GB/s",
                          frac=round(gbs10 / HBM_GBPS, 5), timing="graph10_ms_per_token (the device's rate)"))
        del cache, cache2, fused, attend
    return dict(live_keys=live, heads=H, context=L, note="one decode step (append + attend in one call), batch 1, "
                "HIP graph replay; algorithmic bytes = live K/V rows + appended rows + q + o", **out)


def measure_backward(wl, q, k, v, o, lse, residue, reps=20, warmup=5):
    """The backward of the workload's mask from the forward's o and lse (pa_attn_bwd over
    64 x 64 tiles: pre-pass, dK/dV and dQ kernels), split into the forward's pieces, each
    in its own basis (SplitBackward: the permuted pieces' tensors gathered and their
    gradients scattered back inside the timed region).  For comparison, the whole mask in
    one pass in the residue-`residue` basis, the tensors relabelled before the timed
    region.  Live FLOP = 8 D per live pair and head (dV, dP, dQ, dK; the recomputed scores
    are not counted)."""
    import torch

    from polyhedral_amd import backward as pbwd
    from polyhedral_amd.perm import residue_perm
    H, L, D = wl.H, wl.L, wl.D
    dop = torch.randn(q.shape, generator=torch.Generator().manual_seed(7)).to(q.dtype).to(q.device)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(reps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / reps

    split = pbwd.SplitBackward(wl.pieces, L, q.device)
    ms = timed(lambda: split.backward(q, k, v, o, lse, dop))
    tiles = split.tiles
    # the whole mask in one pass, in one basis
    p = residue_perm(L, residue) if residue else None
    pt = torch.from_numpy(p).long().to(q.device) if p is not None else None
    qp, kp, vp, op, dp = ((x[:, pt].contiguous() if pt is not None else x) for x in (q, k, v, o, dop))
    lsep = lse[:, pt].contiguous() if pt is not None else lse
    single = pbwd.BackwardPlan(wl.union, L, q.device, perm=p)
    ms1 = timed(lambda: single.backward(qp, kp, vp, op, lsep, dp))
    live = int(split.live)
    fl = 8 * D * live * H
    tf = fl / (ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[_dt(q.dtype)]
    return dict(pieces=[(f"rp{s}" if s else "identity") for s, _, _ in split.steps], tile=64, tiles=tiles,
                ms=round(ms, 4), live_tflops=round(tf, 2),
                tile_tflops=round(8 * D * tiles * 64 * 64 * H / (ms * 1e-3) / 1e12, 2),
                roofline=dict(bound="mfma", achieved=round(tf, 2), peak=peak, unit="TFLOP/s", frac=round(tf / peak, 4)),
                single_basis=dict(basis=f"rp{residue}" if residue else "identity", tiles=int(single.kv_num.sum()),
                                  ms=round(ms1, 4), live_tflops=round(fl / (ms1 * 1e-3) / 1e12, 2)),
                note="backward of the whole mask from the forward's o and lse, split into the forward's pieces "
                     "(gathers and scatters of the permuted pieces included); live FLOP = 8 D per live pair and "
                     "head, recomputed scores not counted")


def cpu_leg(wl, o, lse, budget_s=12.0, parity_rows=24, seed=11):
    """The CPU baseline and the parity check, after the timed region.

    cpu_baseline: the oracle's dense masked fp32 attention (gpu/reference.py:5-13 on
    torch, the host's cores) over (head, chunk-row) units of the same inputs, in order,
    until `budget_s` is spent; live-FLOP TFLOP/s over what was processed.
    parity: the timed forward's output `o` (and `lse`) at `parity_rows` sampled query
    rows of EVERY head against the oracle's float64 dense attention of those rows."""
    import torch

    from oracle import attention as oatt
    from oracle import masks as om
    spec = om.NAMED[ORACLE_NAME[wl.name]]
    q, k, v = wl.inputs(0, "cpu")
    qf, kf, vf = (x.float() for x in (q, k, v))
    chunk = 1024 if wl.L <= 32768 else 512
    chunk = min(chunk, wl.L)
    units = [(h, r0) for h in range(wl.H) for r0 in range(0, wl.L, chunk)]
    live = 0
    done = 0
    t0 = time.perf_counter()
    for h, r0 in units:
        r1 = min(wl.L, r0 + chunk)
        rows = om.rows(spec, r0, r1, wl.L)
        oatt.dense_attention_torch(qf[h:h + 1, r0:r1].contiguous(), kf[h:h + 1], vf[h:h + 1],
                                   lambda a, b, rows=rows: rows[a:b], row_chunk=chunk)
        live += int(rows.sum())
        done += 1
        if time.perf_counter() - t0 > budget_s:
            break
    t = time.perf_counter() - t0
    tflops = 4 * wl.D * live / t / 1e12
    base = dict(value=round(tflops, 6), unit="TFLOP/s", cores=torch.get_num_threads(), kind="port",
                sample=f"{done} of {len(units)} (head, {chunk}-row) units of the same inputs, dense masked "
                       f"fp32 attention over all {wl.L} keys (oracle, torch on the host), {t:.1f} s; "
                       f"live pairs in the sample {live}")
    # parity of the timed output: sampled rows (the first and last rows, block edges, random)
    rng = np.random.default_rng(seed)
    fixed = [0, 1, 127, 128, wl.L // 2, wl.L - 1]
    rows = np.array(sorted(set(fixed) | set(rng.integers(0, wl.L, parity_rows - len(fixed)).tolist())))
    ws, wl_ = [], []
    for h in range(wl.H):
        want, wlse = oatt.dense_attention(qf[h:h + 1, rows].numpy(), kf[h:h + 1].numpy(), vf[h:h + 1].numpy(),
                                          lambda a, b: om.live(spec, rows[a:b, None].astype(np.int64),
                                                               np.arange(wl.L)[None, :]),
                                          row_chunk=len(rows))
        ws.append(want[0])
        wl_.append(wlse[0])
    want = np.stack(ws)
    wlse = np.stack(wl_)
    got = o[:, rows].float().cpu().numpy().astype(np.float64)
    err = np.abs(got - want)
    glse = lse[:, rows].cpu().numpy().astype(np.float64)
    fin = np.isfinite(wlse)
    lse_ok = bool(np.array_equal(np.isfinite(glse), fin))
    lse_err = float(np.abs(glse[fin] - wlse[fin]).max()) if fin.any() else 0.0
    tol = {"f32": (1e-5, None), "bf16": (2e-2, 2e-3), "f16": (3e-3, None)}[_dt(wl.dtype)]
    ok = err.max() <= tol[0] and (tol[1] is None or err.mean() <= tol[1]) and lse_ok
    parity = dict(max_abs=float(err.max()), mean_abs=float(err.mean()), lse_max_abs=lse_err,
                  rows=int(len(rows)), heads=wl.H, tol_max=tol[0], tol_mean=tol[1], within_tolerance=bool(ok),
                  reference="oracle float64 dense masked attention (gpu/reference.py:5-13) of the sampled rows "
                            "over all keys, every head; the output is the timed forward's")
    return base, parity


def cpu_index_baseline(wl, pieces, gpu_ms, threads=None):
    """The same pieces' block indices from the oracle's streaming C builder on the host
    (tile classification by predicate evaluation at every (query, key) pair, then the
    compaction of gpu/blockindex.py:32-51), against the device build's wall time.  The
    device build also writes the element bitmaps and the streaming kernel's step
    descriptors, which the host builder does not."""
    from oracle import blockindex as obi
    from polyhedral_amd.perm import residue_perm
    threads = threads or min(16, os.cpu_count() or 1)
    t0 = time.perf_counter()
    for p in pieces:
        perm = residue_perm(wl.L, p.residue) if p.residue else p.perm
        perm = None if perm is None else np.asarray(perm.cpu() if hasattr(perm, "cpu") else perm, dtype=np.int32)
        obi.build(p.mask.terms(), wl.L, p.BQ, p.A, perm_q=perm, perm_kv=perm, threads=threads)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    return dict(gpu_ms=gpu_ms, cpu_ms=round(cpu_ms, 2), speedup=round(cpu_ms / gpu_ms, 2), cpu_threads=threads,
                note="device: SplitPlan construction (classification, compaction, element bitmaps, step "
                     "descriptors, host orchestration), second build in the process; host: oracle C "
                     "builder (classification + compaction) over the same pieces")


def _measured_traffic(workload):
    """HBM bytes per step of the committed counter summary
    (profiles/attn_traffic_<workload>.json: FETCH_SIZE + WRITE_SIZE per dispatch, each
    scaled by what the counter reads for a plain copy of known size) with its source,
    or None if that workload has no summary.  It is not measured in this run."""
    path = os.path.join(ROOT, "profiles", f"attn_traffic_{workload}.json")
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        t = json.load(f)
    src = (f"profiles/attn_traffic_{workload}.json (rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, "
           f"{t.get('kernel', '?')}, measured at commit {t.get('measured_at_commit', '?')})")
    return t.get("hbm_bytes_per_step"), src


def settle(launches, min_ms):
    """Run forwards back to back until `min_ms` of wall time have passed, so the timed
    steps start on settled clocks (over the first ~100 ms of load the GPU's clocks are
    still rising, and a few warmup steps time that ramp).  Returns (ms, forwards)."""
    import torch
    t0 = time.perf_counter()
    n = 0
    while True:
        for _ in range(5):
            for launch in launches:
                launch()
        n += 5
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3
        if ms >= min_ms:
            return ms, n


def algorithmic_bytes(wl, esz):
    """The problem's algorithmic HBM bytes per forward: Q, K and V read once, O written
    once (4 x H x L x D elements), whatever the decomposition."""
    return 4 * wl.H * wl.L * wl.D * esz


def split_bytes(plan, wl, esz):
    """Per launch of the plan, the bytes the decomposition as built must move at least:
    Q, K and V rows read once, O and LSE written once; a piece that merges into a
    previous piece's result also reads that O and LSE once.  Above algorithmic_bytes
    when the plan has several passes (each re-reads Q, K and V, and the merge reads
    the previous output back)."""
    t = wl.H * wl.L * wl.D * esz
    lse = wl.H * wl.L * 4
    out = []
    first = True
    for pieces in plan.launched:
        rd = 3 * t + (t + lse if not first else 0)
        out.append(dict(read=rd, write=t + lse))
        first = False
    return out


def roofline(flops, nbytes, seconds, dt):
    """Both roofline fractions of `flops` live FLOP moving `nbytes` algorithmic bytes in
    `seconds`; the bound is the one the arithmetic intensity selects against the ridge
    (peak FLOP/s over 8 TB/s)."""
    peak = PEAK_TFLOPS[dt]
    ridge = peak * 1e12 / (HBM_GBPS * 1e9)
    inten = flops / nbytes if nbytes else float("inf")
    tf = flops / seconds / 1e12
    gbs = nbytes / seconds / 1e9
    mfma = dict(achieved=round(tf, 3), peak=peak, unit="TFLOP/s", frac=round(tf / peak, 4))
    hbm = dict(achieved=round(gbs, 1), peak=HBM_GBPS, unit="GB/s", frac=round(gbs / HBM_GBPS, 4),
               algorithmic_bytes=int(nbytes))
    bound = "mfma" if inten >= ridge else "hbm"
    return bound, round(inten, 1), round(ridge, 1), mfma, hbm


def run(name, steps, warmup, with_cpu=True, variant=None, device="cuda:0", extras=True, settle_ms=500.0,
        cpu_budget=12.0):
    import torch

    from polyhedral_amd import workloads
    from polyhedral_amd.split import SplitPlan
    wl = workloads.make(name)
    pieces = wl.variants[variant] if variant else wl.pieces
    dev = torch.device(device)
    # the first build also loads the index kernels' code objects; the second is the cost
    # of building a plan in a running process
    build_ms = []
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        plan = SplitPlan(pieces, wl.L, dev)
        torch.cuda.synchronize()
        build_ms.append((time.perf_counter() - t0) * 1e3)
    q, k, v = wl.inputs(0, dev)
    launches, o, lse = plan.prepare(q, k, v)
    s_ms, s_n = settle(launches, settle_ms)
    wall_ms, per_launch = measure(launches, steps, warmup)
    extras = extras and variant is None
    graph_ms = measure_graph(launches)
    iso_ms = measure_isolated(launches, max(25, min(steps, 100))) if extras else None
    residues = [b["piece"].residue for b in plan.built if b["piece"].residue]
    permute = measure_permute(q, k, v, residues[0]) if residues and extras else None
    decode = (measure_decode(wl, q, k, v, (0,) + tuple(sorted(set(residues))))
              if extras and wl.D in (64, 128) and wl.dtype != torch.float32 else None)
    if extras or with_cpu:
        # the timed output, restored after the extra measurements (the decode and backward
        # legs do not write o / lse, but the isolated forwards rewrite them identically)
        for launch in launches:
            launch()
        torch.cuda.synchronize()
    backward = (measure_backward(wl, q, k, v, o, lse, max(residues) if residues else 0)
                if extras and wl.D in (64, 128) and wl.dtype != torch.float32 and wl.L % 64 == 0 else None)
    kernels = [{"run": "attn_run_kernel", "split": "attn_run_kernel (split)", "stream": "attn_stream_kernel",
                "split-grid": "attn_stream_kernel (split)", "wsplit": "attn_wsplit_kernel"}.get(x.kernel, "attn_fwd_kernel")
               for x in launches]
    per = [0.0] * len(plan.built)       # per piece; an empty piece has no launch
    piece_kernel = [None] * len(plan.built)
    for i, pcs in enumerate(plan.launched):
        for bi in pcs:
            # a launch of several pieces is attributed to them by live pairs
            share = plan.built[bi]["live"] / max(1, sum(plan.built[x]["live"] for x in pcs))
            per[bi] = per_launch[i] * share
            piece_kernel[bi] = kernels[i]
    if hasattr(plan, "check"):
        plan.check()
    live = plan.live
    flops_live = 4 * wl.D * live * wl.H
    flops_tile = 4 * wl.D * plan.elements * wl.H
    kern_ms = sum(per)
    dt = _dt(wl.dtype)
    peak = PEAK_TFLOPS[dt]
    achieved = flops_live / (kern_ms * 1e-3) / 1e12
    nbytes = algorithmic_bytes(wl, q.element_size())
    bound, inten, ridge, mfma, hbm = roofline(flops_live, nbytes, kern_ms * 1e-3, dt)
    sb = split_bytes(plan, wl, q.element_size())
    sbytes = sum(x["read"] + x["write"] for x in sb)
    split_hbm = dict(bytes=int(sbytes), per_launch=sb,
                     achieved=round(sbytes / (kern_ms * 1e-3) / 1e9, 1), peak=HBM_GBPS, unit="GB/s",
                     frac=round(sbytes / (kern_ms * 1e-3) / 1e9 / HBM_GBPS, 4),
                     note="bytes the decomposition as built must move at least (each pass reads Q, K, V; "
                          "a merging pass also reads the previous O and LSE), over the kernel time")
    res = dict(
        workload=name + (f"[{variant}]" if variant else ""), description=wl.description, dtype=dt,
        H=wl.H, L=wl.L, D=wl.D, live_pairs_per_head=live, tile_elements_per_head=plan.elements,
        waste=round(plan.elements / live, 4) if live else None,
        pieces=[dict(mask=b["piece"].mask.name, BQ=b["piece"].BQ, A=b["piece"].A,
                     basis="identity" if b["perm"] is None else "permuted", tiles=b["tiles"], live=b["live"],
                     kernel=piece_kernel[i],
                     launch_ms=round(per[i], 5),
                     live_tflops=round(4 * wl.D * b["live"] * wl.H / (per[i] * 1e-3) / 1e12, 2) if per[i] else None)
                for i, b in enumerate(plan.built)],
        index_build_ms=round(build_ms[1], 2), index_build_cold_ms=round(build_ms[0], 2),
        settle_ms=round(s_ms, 1), settle_forwards=s_n,
        ms_per_step=round(wall_ms, 5), kernel_ms=round(kern_ms, 5),
        live_tflops=round(flops_live / (wall_ms * 1e-3) / 1e12, 3),
        kernel_live_tflops=round(achieved, 3), tile_tflops=round(flops_tile / (kern_ms * 1e-3) / 1e12, 3),
        peak_tflops=peak, frac_peak=round(achieved / peak, 4),
        bound=bound, intensity_flop_per_byte=inten, ridge_flop_per_byte=ridge, mfma=mfma, hbm=hbm,
        split_hbm=split_hbm,
        min_hbm_bytes=nbytes,
    )
    res["hbm_floor_ms"] = round(res["min_hbm_bytes"] / (HBM_GBPS * 1e9) * 1e3, 5)
    gb, _, _, gmfma, ghbm = roofline(flops_live, nbytes, graph_ms * 1e-3, dt)
    res["graph"] = dict(ms_per_step=round(graph_ms, 5), live_tflops=gmfma["achieved"], mfma_frac=gmfma["frac"],
                        hbm_frac=ghbm["frac"],
                        protocol="10 forwards captured in one HIP graph, replayed back to back (the device's "
                                 "rate; a forward of a few microseconds is otherwise paced by the host's "
                                 "launches), median of 3 rounds of >= 50 ms")
    if iso_ms is not None:
        res["isolated"] = dict(ms_median=round(iso_ms, 5),
                               live_tflops=round(flops_live / (iso_ms * 1e-3) / 1e12, 3),
                               protocol="one forward per event pair after zeroing a 512 MiB buffer, device "
                                        "synchronised between forwards, median (gpu/bench.py:11-24 with a flush "
                                        "larger than the memory-side cache)")
    res["permute"] = permute
    res["decode"] = decode
    res["backward"] = backward
    res["_launches"] = len(launches)
    if with_cpu:
        log(f"[bench] cpu baseline and parity for {res['workload']} ...")
        res["cpu_baseline"], res["parity"] = cpu_leg(wl, o, lse, budget_s=cpu_budget)
        if extras:
            res["index_build"] = cpu_index_baseline(wl, pieces, res["index_build_ms"])
    del launches, o, lse, q, k, v, plan
    torch.cuda.empty_cache()
    return res


def brief(r):
    """The per-workload entry of the bench line."""
    out = dict(workload=r["workload"], dtype=r["dtype"], H=r["H"], L=r["L"], D=r["D"],
               pieces=[f"{p['mask']} {p['BQ']}x{p['A']} {p['basis']}" for p in r["pieces"]],
               ms_per_step=r["ms_per_step"], kernel_ms=r["kernel_ms"], live_tflops=r["live_tflops"],
               roofline=dict(bound=r["bound"], intensity_flop_per_byte=r["intensity_flop_per_byte"],
                             ridge_flop_per_byte=r["ridge_flop_per_byte"], mfma=r["mfma"], hbm=r["hbm"]),
               split_hbm=dict(bytes=r["split_hbm"]["bytes"], frac=r["split_hbm"]["frac"]),
               graph=r["graph"], waste=r["waste"], settle_ms=r["settle_ms"])
    for key in ("parity", "cpu_baseline"):
        if key in r:
            out[key] = r[key]
    return out


def log_result(r):
    log(f"[bench]   {r['ms_per_step']:.4f} ms/step  kernel {r['kernel_ms']:.4f} ms  "
        f"{r['kernel_live_tflops']:.1f} live TFLOP/s (mfma {100 * r['mfma']['frac']:.1f}%, "
        f"hbm {100 * r['hbm']['frac']:.1f}% of algorithmic bytes; {r['bound']}-bound; split bytes at "
        f"{100 * r['split_hbm']['frac']:.1f}% of HBM)  waste {r['waste']}  graph {r['graph']['ms_per_step']:.4f} ms")
    if r.get("parity"):
        pr = r["parity"]
        log(f"[bench]   parity: max {pr['max_abs']:.2e} mean {pr['mean_abs']:.2e} over {pr['rows']} rows x "
            f"{pr['heads']} heads ({'ok' if pr['within_tolerance'] else 'OUT OF TOLERANCE'})")
    if r.get("isolated"):
        log(f"[bench]   isolated {r['isolated']['ms_median']:.4f} ms ({r['isolated']['live_tflops']:.1f} TFLOP/s)")
    if r.get("index_build"):
        ib = r["index_build"]
        log(f"[bench]   index build: device {ib['gpu_ms']:.2f} ms, host C builder {ib['cpu_ms']:.1f} ms "
            f"on {ib['cpu_threads']} threads ({ib['speedup']:.0f}x)")
    if r.get("decode"):
        dd = r["decode"]
        log("[bench]   decode (append + attend in one call, 1 token): " + ", ".join(
            f"{b} {dd[b]['ms_per_token'] * 1e3:.1f} us ({dd[b]['gb_per_s']:.0f} GB/s; 10-step graph "
            f"{dd[b]['graph10_ms_per_token'] * 1e3:.1f} us; as two calls "
            f"{dd[b]['separate_ms_per_token'] * 1e3:.1f} / {dd[b]['separate_graph10_ms_per_token'] * 1e3:.1f} us)"
            for b in dd if isinstance(dd[b], dict)))
    if r.get("backward"):
        bw = r["backward"]
        sb = bw["single_basis"]
        log(f"[bench]   backward ({' + '.join(bw['pieces'])}, 64x64, {bw['tiles']} tiles): {bw['ms']:.3f} ms, "
            f"{bw['live_tflops']:.0f} live TFLOP/s ({100 * bw['roofline']['frac']:.1f}%); one pass in "
            f"{sb['basis']} ({sb['tiles']} tiles): {sb['ms']:.3f} ms")
    if r.get("permute"):
        pm_ = r["permute"]
        log(f"[bench]   permute rp{pm_['residue']}: Q/K/V gather {pm_['gather_qkv']['gb_per_s']:.0f} GB/s, "
            f"O scatter {pm_['scatter_o']['gb_per_s']:.0f} GB/s")


# the other workloads of the default run: (workload, decomposition variant or None)
CONFIGS = [("window128-L1k", None), ("dilated8-L8k", None), ("dilated8-L8k", "identity"),
           ("bandlat-L16k", "16x16"), ("sinkwin-L32k", None), ("prefixlat-L64k", None), ("bandlat32-L64k", None)]


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--settle-ms", type=float, default=500.0,
                    help="wall time of back-to-back forwards before the warmup and the timed steps")
    ap.add_argument("--workload", default=None)
    ap.add_argument("--variant", default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="only the headline workload")
    ap.add_argument("--forward-only", action="store_true",
                    help="time only the forward of the workload (no isolated, permute, decode or backward legs)")
    ap.add_argument("--all", action="store_true")
    ap.add_argument("--report", default=None)
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only copy a MIB-sized device buffer a few times (the known-size kernel that "
                         "scales the FETCH_SIZE / WRITE_SIZE counters), then exit")
    a = ap.parse_args()
    if a.steps < 1 or a.warmup < 0:
        ap.error(f"--steps must be >= 1 and --warmup >= 0 (got {a.steps}, {a.warmup})")
    if a.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {a.gpus}). "
              "The attention shards over heads with no exchange; run one process per GPU.", file=sys.stderr)
        sys.exit(2)
    import torch
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if a.copy_calibration:
        n = a.copy_calibration * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.int32, device="cuda")
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps(dict(copy_calibration_bytes=n * 4, launches=3)))
        return
    from polyhedral_amd import workloads

    if a.all:
        rows = []
        for name in workloads.NAMES:
            wl = workloads.make(name)
            for variant in [None] + list(wl.variants):
                log(f"[bench] {name} {variant or ''}")
                rows.append(run(name, a.steps, a.warmup, with_cpu=not a.no_cpu and variant is None,
                                variant=variant, settle_ms=a.settle_ms))
                log_result(rows[-1])
        out = dict(device=torch.cuda.get_device_name(0), results=rows)
        if a.report:
            with open(a.report, "w") as f:
                json.dump(out, f, indent=1)
        print(json.dumps(out))
        return

    name = a.workload or workloads.HEADLINE
    log(f"[bench] {name} {a.variant or ''}")
    r = run(name, a.steps, a.warmup, with_cpu=not a.no_cpu, variant=a.variant, settle_ms=a.settle_ms,
            extras=not a.forward_only)
    log_result(r)
    configs = []
    if not a.no_configs and a.workload is None:
        for cname, variant in CONFIGS:
            log(f"[bench] {cname} {variant or ''}")
            rc = run(cname, a.steps, a.warmup, with_cpu=not a.no_cpu, variant=variant, extras=False,
                     settle_ms=min(a.settle_ms, 300.0), cpu_budget=3.0)
            log_result(rc)
            configs.append(brief(rc))
    wl = workloads.make(name)
    traffic, traffic_src = _measured_traffic(r["workload"])
    main_roof = r["mfma"] if r["bound"] == "mfma" else r["hbm"]
    line = dict(
        metric=METRIC, value=r["live_tflops"], unit="TFLOP/s", n_gpus=1, steps=a.steps, warmup=a.warmup,
        ms_per_step=r["ms_per_step"], higher_is_better=True, scaling="weak", vs_baseline=None,
        dtype=r["dtype"], data="synthetic",
        config=dict(workload=r["workload"], description=wl.description, L=wl.L, H=wl.H, D=wl.D, B=1,
                    live_pairs_per_head=r["live_pairs_per_head"], waste=r["waste"],
                    pct_bf16_peak=round(100 * r["live_tflops"] / PEAK_TFLOPS["bf16"], 2),
                    pieces=r["pieces"], index_build_ms=r["index_build_ms"]),
        settle_ms=r["settle_ms"], settle_forwards=r["settle_forwards"],
        roofline=dict(bound=r["bound"], achieved=main_roof["achieved"], peak=main_roof["peak"],
                      unit=main_roof["unit"], frac=main_roof["frac"], traffic=traffic,
                      traffic_unit="HBM bytes per step (all launches of one step)", traffic_source=traffic_src,
                      intensity_flop_per_byte=r["intensity_flop_per_byte"],
                      ridge_flop_per_byte=r["ridge_flop_per_byte"], mfma=r["mfma"], hbm=r["hbm"],
                      split_hbm=r["split_hbm"],
                      kernel=" + ".join(sorted({p["kernel"] for p in r["pieces"] if p["kernel"]})) +
                             " (all launches of one step, durations from HIP events on the launch stream"
                             " around each launch of every fourth timed step; a bracket also holds its own"
                             " event record, so the launches' sum can exceed the wall time per step)",
                      algorithmic="live FLOP = 4 * D * live pairs * heads; algorithmic bytes = Q, K, V read "
                                  "once and O written once per forward (4 * H * L * D elements); the bound is "
                                  "the one their ratio selects against the ridge (peak FLOP/s over 8 TB/s). "
                                  "split_hbm: the bytes the two-pass split as built must move at least"),
        graph=r["graph"],
        parity=r.get("parity"),
        cpu_baseline=r.get("cpu_baseline"),
        configs=configs,
        index_build=r.get("index_build"),
        isolated=r.get("isolated"),
        permute=r["permute"],
        decode=r["decode"],
        backward=r["backward"],
    )
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
