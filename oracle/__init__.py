"""CPU oracle for the sparse 3-D refiner step -- TEST INFRASTRUCTURE ONLY.

A NumPy restatement of the reference's algorithm for the hot path, each function citing the reference file:line it
follows. It is the checker, never the thing measured or shipped: only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it. The product (promptmoge_amd) never imports it and has no CPU fallback.

Modules
  numerics   bit-reproducible fp32 exp/log/SiLU/quantise, the same operation sequence as the kernels' pmg_math.h
  structure  voxelisation (v3.py:305-344), kernel offsets (_core.py:65-82), linearisation (_core.py:89-102),
             column map (_core.py:269-295), sorted map (_core.py:105-124, 298-304), brute-force map, tile masks,
             compacted per-tap kernel maps (_core.py:430-437)
  conv       submanifold conv: exact integer accumulation, the deployed int8 epilogues (SparseConvInt8.metal,
             qat.py), and the fp32 _fallback order (_core.py:399-441)
  fit        fit_scale_shift (prompt_stem.py:211-240): fp64-sum form (what the kernel computes) and the literal fp32
             form of the reference
  fill       nearest_fill (promptmoge/model.py:61-72): the exact EDT feature transform in two separable passes
  pool       build_pool_cache / sparse_pool / sparse_upsample (_core.py:339-505): perfect-partition pooling with
             sorted unique output keys, mean/sum in input order, nearest upsampling by parent
  gauge      prompt_gauge_poly (v3.py:151-183): pooled inputs, IRLS with the lower median, exp(poly) correction
  blocks     the int8 contract (qat.py:28-57, Refiner.swift:147-148), the residual block (flex_sparse_blocks.py:70-75)
             and linear layers in three arithmetics: the reference's fp32, its QAT fake-quant, the deployed int8
  refiner    the fused step (v3.py:346-383, 547-576; sparse_unet.py:176-258 single level; flex_sparse_blocks.py:70-75)
             in the deployed int8 / fp16 arithmetic, and the reference's fp32 fake-quant (QAT) formulation; the refine
             loop's output gate and elastic anchor (v3.py:565-573)
  unet       the multi-level Sparse3DUNet (sparse_unet.py:176-258; PoolDown / NearestUp, flex_sparse_blocks.py:78-105):
             level structure, encoder conditioning, fuse_proj, per-level stages, in the three arithmetics

What pins each function (golden vectors, closed forms, brute force, invariants) is listed in tests/test_oracle*.py.
The reference ships no golden vectors or tests for this path; tests/golden/refiner_vectors.npz holds vectors its own
modules produced (tests/golden/make_refiner_vectors.py), for the composition nothing else pins.
"""
