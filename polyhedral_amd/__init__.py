"""MI355X-native (gfx950) block-sparse masked attention forward, polyattn call surface.

Subpackages and modules:
  polyhedral_amd.gpu        drop-in modules named as the reference's gpu/ directory
                            (blockindex, permute, triton_attn, masks_gpu, reference,
                            bench, launchsweep) plus split (disjoint split + LSE merge)
  polyhedral_amd.polyattn   mask zoo and element-count model (polyattn.masks / cost)
  polyhedral_amd.spec       mask predicate -> device predicate terms
  polyhedral_amd.index      GPU block-index builder
  polyhedral_amd.perm       GPU class-A permutation
  polyhedral_amd.attention  GPU attention forward
  polyhedral_amd.split      disjoint split + log-sum-exp merge
"""
__all__ = ["attention", "index", "perm", "spec", "split"]
