"""rfill: the RidgeFill late-layer fill on MI355X (gfx950).

Python host code mirroring the reference's code/kva fill API (Arm, Projector, fill / fill_kv over
explicit caches) on PyTorch-ROCm tensors, with the arithmetic in librfill.so's hand-written HIP
kernels (the C ABI in include/rfill.h). Submodules:
  rfill.ops    tensor front end of the C ABI
  rfill.model  FillModel: packed per-layer weights and the fill / fill_kv API
  rfill.kva    Arm, Projector, fill_late (finish()'s late-layer fill loop)
  rfill.synth  seeded synthetic workloads
Importing rfill does not load the library; the first kernel call does, and raises ImportError if
librfill.so is not built (there is no CPU fallback).
"""
__version__ = "0.1.0"
