"""hi3d_amd — the Hi3D refiner's sparse-tensor hot path on MI355X (gfx950).

Voxel-hash kernel maps, gather-MFMA sparse convolution (submanifold 3^3, 2x2x2/s2 and
its transpose), the W8A8 int8 linear and the LayerNorm + adaLN row kernel, as
hand-written HIP kernels behind a C ABI (``include/hi3d_amd.h``), with the reference's
Python call surfaces on top:

* :mod:`hi3d_amd.spconv` — the spconv 2.3.6 subset (``SubMConv3d``,
  ``SparseConvTensor``, ``ops.get_indice_pairs``, ``core.IndiceData``, ...);
  :func:`hi3d_amd.spconv.install` registers it as ``spconv``;
* :mod:`hi3d_amd.sparse_backend` — ``sparc3d.ops.sparse_backend``;
* :mod:`hi3d_amd.nn` — ``SparseTensor``, ``SparseConv3d``, ``SparseDownsample``,
  ``SparseUpsample``;
* :mod:`hi3d_amd.sparse` — the MLX backend's ``neighbour_table`` / ``Level`` /
  ``sparse_conv`` / ``downsample_structure`` / ``child_neighbour_table``;
* :mod:`hi3d_amd.w8a8` — ``signs``, ``quantize_activation``, ``linear``;
* :mod:`hi3d_amd.kernels` — ``layer_norm_modulate``.

Every operation runs on the GPU; there is no host fallback.
"""

__version__ = "0.1.0"
