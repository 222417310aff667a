"""The five benchmark workloads of this path, as split plans.

Each workload is a mask over L positions, a head count, a head dimension, an
element type and a decomposition into disjoint pieces (mask, tile shape, basis).
A piece in a residue-class basis (class-A permutation rp-s, gpu/permute.py:12-15)
reads Q/K/V through the permutation inside the kernel.

  window128-L1k     causal sliding window 128, fp32, H=4, L=1024, D=64, tiles 128x128
  dilated8-L8k      (q-kv) % 8 == 0, bf16, H=16, L=8192, D=128, tiles 128x32, basis rp8
  bandlat-L16k      0 <= q-kv < 256 or (q-kv) % 16 == 0, bf16, H=32, L=16384, D=128:
                    band-256 (identity, 128x32) + lattice-16 minus band (rp16, 128x32)
  sinkwin-L32k      kv <= q and (kv < 64 or q-kv < 1024), bf16, H=32, L=32768, D=128,
                    tiles 128x32, k scaled x4 on the first 64 keys
  prefixlat-L64k    prefix-LM 2048 + (lattice-32 minus prefix-LM) (empty), bf16, H=8,
                    L=65536, D=128, tiles 128x32, one pass per sub-mask
  bandlat32-L64k    the non-degenerate companion at the prefix-LM workload's shape (H=8,
                    L=65536, D=128, bf16), whose second sub-mask is not empty, so the
                    log-sum-exp combine of two passes runs at L = 65536:
                    0 <= q-kv < 256 or (q-kv) % 32 == 0, split into band-256 (identity,
                    128x32) + lattice-32 minus band (rp32, 128x32)

bandlat-L16k also has the variant "16x16": the same two pieces on their 16x16-floor
block indices (the general kernel, one 16-row wave per query block).
"""
from dataclasses import dataclass, field

import torch

from .polyattn import masks as M
from .split import Piece


@dataclass
class Workload:
    name: str
    description: str
    H: int
    L: int
    D: int
    dtype: torch.dtype
    pieces: list
    union: object                 # the whole mask (the union of the pieces)
    k_scale_first: tuple = None   # (n, factor): k[:, :n] *= factor before the cast
    variants: dict = field(default_factory=dict)  # alternative decompositions (name -> pieces)

    def inputs(self, seed=0, device="cpu"):
        """CPU torch.Generator(seed): q, k, v drawn as fp32 randn [H, L, D], then cast."""
        g = torch.Generator().manual_seed(seed)
        q, k, v = (torch.randn(self.H, self.L, self.D, generator=g) for _ in range(3))
        if self.k_scale_first is not None:
            n, f = self.k_scale_first
            k[:, :n] *= f
        return tuple(x.to(self.dtype).to(device) for x in (q, k, v))


def make(name):
    if name == "window128-L1k":
        m = M.SlidingWindow(128)
        return Workload(name, "causal sliding window 128, fp32, H=4, L=1024, D=64, 128x128 tiles",
                        4, 1024, 64, torch.float32, [Piece(m, 128, 128)], m,
                        variants={"16x16": [Piece(m, 16, 16)]})
    if name == "dilated8-L8k":
        m = M.Dilated(8)
        L = 8192
        return Workload(name, "dilated-8 lattice, bf16, H=16, L=8192, D=128, 128x32 tiles, rp8 basis",
                        16, L, 128, torch.bfloat16, [Piece(m, 128, 32, residue=8)], m,
                        variants={"identity": [Piece(m, 128, 32)]})
    if name == "bandlat-L16k":
        L = 16384
        band = M.SlidingWindow(256)
        lat = M.Difference(M.Dilated(16), band)
        union = M.LocalStrided(256, 16)
        return Workload(name, "band-256 | lattice-16, bf16, H=32, L=16384, D=128: band (identity, 128x32) "
                              "+ lattice-16 minus band (rp16, 128x32), LSE merge",
                        32, L, 128, torch.bfloat16, [Piece(band, 128, 32), Piece(lat, 128, 32, residue=16)],
                        union, variants={"single-rp16": [Piece(union, 128, 32, residue=16)],
                                         "16x16": [Piece(band, 16, 16), Piece(lat, 16, 16, residue=16)]})
    if name == "sinkwin-L32k":
        m = M.SinksWindow(64, 1024)
        return Workload(name, "64 sinks + causal window 1024, bf16, H=32, L=32768, D=128, 128x32 tiles",
                        32, 32768, 128, torch.bfloat16, [Piece(m, 128, 32)], m, k_scale_first=(64, 4.0))
    if name == "prefixlat-L64k":
        L = 65536
        p = M.PrefixLM(2048)
        sub2 = M.Difference(M.Dilated(32), p)
        return Workload(name, "prefix-LM 2048 + (lattice-32 minus prefix-LM), bf16, H=8, L=65536, D=128, "
                              "128x32 tiles, one pass per sub-mask",
                        8, L, 128, torch.bfloat16, [Piece(p, 128, 32), Piece(sub2, 128, 32, residue=32)],
                        M.Union(p, M.Dilated(32)))
    if name == "bandlat32-L64k":
        L = 65536
        band = M.SlidingWindow(256)
        lat = M.Difference(M.Dilated(32), band)
        return Workload(name, "band-256 | lattice-32, bf16, H=8, L=65536, D=128: band (identity, 128x32) "
                              "+ lattice-32 minus band (rp32, 128x32), LSE merge (the two-pass companion at "
                              "the prefix-LM workload's shape)",
                        8, L, 128, torch.bfloat16, [Piece(band, 128, 32), Piece(lat, 128, 32, residue=32)],
                        M.LocalStrided(256, 32))
    raise KeyError(name)


NAMES = ["window128-L1k", "dilated8-L8k", "bandlat-L16k", "sinkwin-L32k", "prefixlat-L64k", "bandlat32-L64k"]
HEADLINE = "bandlat-L16k"
