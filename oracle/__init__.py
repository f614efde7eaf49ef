"""CPU oracle of the Hi3D sparse hot path — TEST INFRASTRUCTURE ONLY.

A NumPy / PyTorch-CPU restatement of the reference's algorithms, used as the checker
of the HIP kernels (by ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg
of ``bench.py``). Nothing in the product package imports, calls or links it; the
product path has no CPU fallback.

Modules and the reference code they restate (file:line in devin-lai/Hi3Dv1.0-mlx):

* :mod:`oracle.kmap` — ``_voxel_keys`` / ``subm_pairs``
  (src/hi3d_mac/torch_backend/sparse_conv.py:109-149), ``neighbour_table`` /
  ``child_neighbour_table`` / ``downsample_structure``
  (src/hi3d_mac/mlx_backend/sparse.py:29-95,217-233).
* :mod:`oracle.conv` — ``subm_conv`` / ``_accumulate``
  (src/hi3d_mac/torch_backend/sparse_conv.py:152-195), the dense ``F.conv3d`` check of
  tests/test_backends.py:32-50, float64 gather sums, and the stride-2 pair's dense
  equivalents (``F.conv3d(stride=2)``, ``F.conv_transpose3d(stride=2)``).
* :mod:`oracle.w8a8` — ``signs`` / ``_QUANT`` / ``_GEMM`` epilogue
  (src/hi3d_mac/mlx_backend/w8a8.py:16-80) and the integer check of
  tests/test_w8a8_inference.py:8-20.
* :mod:`oracle.norm` — ``layer_norm_modulate`` (src/hi3d_mac/mlx_backend/kernels.py:
  162-201) and the residual block (src/sparc3d/models/transformers/
  sparc3d_transformer.py:132-144; src/hi3d_mac/mlx_backend/transformer.py:413-437).
* :mod:`oracle.baseline` — the reference's CPU fallback (sort + searchsorted map,
  per-offset gather / matmul / ``index_add_``), timed as the CPU baseline.

How each function is pinned (golden vectors, closed forms, brute force, library
routines) is listed in ``tests/test_oracle.py``; every function has such a check.
"""
