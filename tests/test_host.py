"""Host-side checks without a GPU: the C-ABI library loads and exports every symbol the
header declares, workspace queries, argument validation in C and Python (errors raised
before any kernel launch), and the spconv module registration."""

from __future__ import annotations

import ctypes
import re
import sys
import types

import pytest
import torch

from conftest import ROOT

HEADER = ROOT / "include" / "hi3d_amd.h"


def _header_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hi3d_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from hi3d_amd import _lib

    lib = _lib.lib()
    declared = _header_functions()
    assert len(declared) >= 20
    for name in declared:
        assert hasattr(lib, name), name
    assert sorted(_lib.exported_symbols()) == declared
    assert lib.hi3d_version().decode().startswith("hi3d_amd")


def test_workspace_queries():
    from hi3d_amd import _lib

    assert _lib.query("hi3d_kmap_workspace", 1000, 0, 0) >= 2048 * 8
    assert _lib.query("hi3d_kmap_workspace", 1000, 0, 1) >= 2048 * 12
    assert _lib.query("hi3d_kmap_workspace", 0, 0, 0) > 0
    with pytest.raises(ValueError, match="power of two"):
        _lib.query("hi3d_kmap_workspace", 10, 100, 0)
    assert _lib.query("hi3d_kmap_pairs_workspace", 1000, 27) > 0
    assert _lib.query("hi3d_conv_plan_workspace", 10**6) > 10**6 * 24
    assert _lib.query("hi3d_downsample_workspace", 10**6) > 10**6 * 24
    assert _lib.query("hi3d_child_table_workspace", 1000) > 8000 * 12
    assert _lib.lib().hi3d_conv_tile_rows() == 128


def test_c_argument_validation_without_launch():
    """Invalid arguments are rejected with HI3D_ERR_INVALID before anything runs."""
    from hi3d_amd import _lib

    lib = _lib.lib()
    null = None
    # even kernel size
    rc = lib.hi3d_kmap_subm(null, 0, 4, 4, 4, 1, 2, 0, null, 0, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "ksize" in _lib.last_error()
    # fp16 rows of 5 channels are not 16-byte aligned for the MFMA path
    rc = lib.hi3d_gather_conv(null, 10, 5, null, null, 8, 27, null, null, null, 10, null, 0, _lib.F16, null, null)
    assert rc == _lib.ERR_INVALID and "16 bytes" in _lib.last_error()
    # float64 is not an MFMA dtype
    rc = lib.hi3d_gather_conv(null, 10, 8, null, null, 8, 27, null, null, null, 10, null, 0, _lib.F64, null, null)
    assert rc == _lib.ERR_INVALID
    # rotation needs K % 64
    rc = lib.hi3d_w8a8_quantize(null, 4, 72, ctypes.c_void_p(16), null, null, null)
    assert rc == _lib.ERR_INVALID and "H64" in _lib.last_error()
    rc = lib.hi3d_w8a8_gemm(null, null, null, null, null, 4, 8, 24, null, null, null)
    assert rc == _lib.ERR_INVALID
    rc = lib.hi3d_layer_norm_modulate(null, 4, 8, 1e-6, ctypes.c_void_p(16), null, null, null, null, null)
    assert rc == _lib.ERR_INVALID
    # the narrow kernel: at most 16 outputs, 64-byte input rows, no float64
    rc = lib.hi3d_gather_conv_narrow(null, 10, 64, null, null, 17, 27, null, null, null, 10, null, 0, _lib.F16, null,
                                     null)
    assert rc == _lib.ERR_INVALID and "1..16 output" in _lib.last_error()
    rc = lib.hi3d_gather_conv_narrow(null, 10, 24, null, null, 8, 27, null, null, null, 10, null, 0, _lib.F16, null,
                                     null)
    assert rc == _lib.ERR_INVALID and "64 bytes" in _lib.last_error()
    rc = lib.hi3d_gather_conv_narrow(null, 10, 64, null, null, 8, 27, null, null, null, 10, null, 0, _lib.F64, null,
                                     null)
    assert rc == _lib.ERR_INVALID
    # unique: key_bits range, row dtypes and widths
    rc = lib.hi3d_unique_keys(null, 10, 64, null, 1 << 20, null, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "key_bits" in _lib.last_error()
    rc = lib.hi3d_pack_rows(null, _lib.F32, 10, 3, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "I32 or I64" in _lib.last_error()
    rc = lib.hi3d_pack_rows(null, _lib.I64, 10, 9, null, null, null, null)
    assert rc == _lib.ERR_INVALID and "1..8" in _lib.last_error()
    # the parent-major transposed conv: fp16 / bf16, cin 64 or 128, cout 64; outputs under 2 GiB
    assert lib.hi3d_stride2_up_supported(128, 64, _lib.F16) == 1 and lib.hi3d_stride2_up_supported(64, 64, _lib.BF16) == 1
    assert lib.hi3d_stride2_up_supported(256, 64, _lib.F16) == 0 and lib.hi3d_stride2_up_supported(128, 128, _lib.F16) == 0
    assert lib.hi3d_stride2_up_supported(128, 64, _lib.F32) == 0
    rc = lib.hi3d_stride2_up_conv(null, 10, 256, null, null, 64, null, 30, _lib.F16, null, null)
    assert rc == _lib.ERR_INVALID and "cin 64 or 128" in _lib.last_error()
    rc = lib.hi3d_stride2_up_conv(null, 10, 128, null, null, 64, null, 1 << 24, _lib.F16, null, null)
    assert rc == _lib.ERR_INVALID and "2 GiB" in _lib.last_error()
    # zero-size calls succeed without touching memory
    assert lib.hi3d_stride2_up_conv(null, 0, 128, null, null, 64, null, 0, _lib.F16, null, null) == 0
    assert lib.hi3d_gather_conv_simple(null, 0, 3, null, null, 5, 27, null, 0, null, 0, _lib.F64, null, null) == 0
    assert lib.hi3d_gather_conv_narrow(null, 0, 64, null, null, 8, 27, null, null, null, 0, null, 0, _lib.F16, null,
                                       null) == 0
    assert lib.hi3d_w8a8_quantize(null, 0, 64, null, null, null, null) == 0
    # resampling factors: positive, product at most 256 (checked before any launch)
    fake = ctypes.c_void_p(16)
    for f in ((0, 2, 2), (2, -1, 2), (8, 8, 8)):
        rc = lib.hi3d_resample_structure(null, 10, 8, 8, 8, 1, *f, null, 0, null, null, null, null, fake, null, null)
        assert rc == _lib.ERR_INVALID and "factors" in _lib.last_error()
    rc = lib.hi3d_resample_down_table(null, null, 10, 4, 257, null, null)
    assert rc == _lib.ERR_INVALID
    # the sorted transposed conv refuses what the row-order one refuses; its plan checks the window
    rc = lib.hi3d_stride2_up_conv_sorted(null, 10, 256, null, null, 64, null, null, 30, _lib.F16, null, null)
    assert rc == _lib.ERR_INVALID and "cin 64 or 128" in _lib.last_error()
    rc = lib.hi3d_stride2_up_plan(fake, 10, 30, 40, null, 0, null, null, null)
    assert rc == _lib.ERR_INVALID and "window_log2" in _lib.last_error()
    assert lib.hi3d_stride2_up_tile_rows() == 32
    # the LayerNorm + activation entry: unknown activation
    rc = lib.hi3d_layer_norm_act(fake, 4, 8, 1e-6, null, null, null, null, 7, fake, null)
    assert rc == _lib.ERR_INVALID and "activation" in _lib.last_error()
    # the LayerNorm + quantise entry: widths, rotation, pairs of vectors, alignment
    lnq = lib.hi3d_layer_norm_quantize
    for c, signs, what in ((12, null, "multiple of 8"), (72, fake, "H64"), (4160, fake, "4096")):
        rc = lnq(fake, 4, c, 1e-6, null, null, null, null, signs, fake, fake, null)
        assert rc == _lib.ERR_INVALID and what in _lib.last_error()
    rc = lnq(fake, 4, 64, 1e-6, fake, null, null, null, null, fake, fake, null)
    assert rc == _lib.ERR_INVALID and "weight and bias" in _lib.last_error()
    rc = lnq(fake, 4, 64, 1e-6, null, null, null, fake, null, fake, fake, null)
    assert rc == _lib.ERR_INVALID and "scale and shift" in _lib.last_error()
    rc = lnq(ctypes.c_void_p(24), 4, 64, 1e-6, null, null, null, null, null, fake, fake, null)
    assert rc == _lib.ERR_INVALID and "aligned" in _lib.last_error()
    rc = lnq(fake, 4, 64, 1e-6, null, null, null, null, null, ctypes.c_void_p(20), fake, null)
    assert rc == _lib.ERR_INVALID and "aligned" in _lib.last_error()
    rc = lnq(fake, 4, 64, 1e-6, null, null, null, null, null, null, fake, null)
    assert rc == _lib.ERR_INVALID and "null" in _lib.last_error()
    assert lnq(null, 0, 64, 1e-6, null, null, null, null, null, null, null, null) == 0
    # the row-wise linear entry: channel counts and alignment
    for cin, cout, what in ((40, 64, "cin"), (144, 64, "cin"), (64, 96, "cout"), (64, 320, "cout")):
        rc = lib.hi3d_dense_linear(fake, 4, cin, fake, null, cout, null, fake, null)
        assert rc == _lib.ERR_INVALID and what in _lib.last_error()
    rc = lib.hi3d_dense_linear(ctypes.c_void_p(24), 4, 64, fake, null, 64, null, fake, null)
    assert rc == _lib.ERR_INVALID and "aligned" in _lib.last_error()
    assert lib.hi3d_dense_linear(null, 0, 64, null, null, 64, null, null, null) == 0
    # the convolution with the fused row norm: 128 outputs, 128..512 inputs in steps of 64
    cln = lib.hi3d_gather_conv_ln_silu
    for cin, cout, what in ((128, 256, "128 output"), (96, 128, "128..512"), (576, 128, "128..512")):
        rc = cln(fake, 10, cin, fake, null, cout, 27, fake, fake, fake, 10, fake, 1, fake, fake, 1e-6, fake, null)
        assert rc == _lib.ERR_INVALID and what in _lib.last_error()
    rc = cln(fake, 10, 128, fake, null, 128, 27, fake, fake, fake, 10, fake, 0, fake, fake, 1e-6, fake, null)
    assert rc == _lib.ERR_INVALID and "batches" in _lib.last_error()
    assert cln(null, 0, 128, null, null, 128, 27, null, null, null, 0, null, 1, null, null, 1e-6, null, null) == 0


def test_python_validation_matches_reference_errors():
    from hi3d_amd import sparse_backend, spconv, w8a8

    with pytest.raises(ValueError, match="kernel_size must be odd"):
        sparse_backend.Conv3d(4, 4, kernel_size=2)
    with pytest.raises(ValueError, match="only stride 1"):
        sparse_backend.Conv3d(4, 4, stride=2)
    with pytest.raises(ValueError, match="submanifold padding"):
        sparse_backend.Conv3d(4, 4, padding=0)
    conv = sparse_backend.Conv3d(4, 6)
    assert sparse_backend.is_sparse_conv(conv) and conv.indice_key == "subm3"
    assert tuple(conv.weight.shape) == (6, 3, 3, 3, 4)
    with pytest.raises(ValueError, match="cubic odd"):
        spconv.SubMConv3d(4, 4, kernel_size=(3, 3, 5))
    with pytest.raises(ValueError, match="grouped"):
        spconv.SubMConv3d(4, 4, groups=2)
    with pytest.raises(NotImplementedError):
        spconv.SparseConv3d(4, 4, kernel_size=3, stride=2)
    with pytest.raises(ValueError, match="indice_key"):
        spconv.SparseInverseConv3d(4, 4, kernel_size=2)
    with pytest.raises(NotImplementedError):
        spconv.get_indice_pairs(torch.zeros((1, 4), dtype=torch.int32), 1, [4, 4, 4], spconv.ConvAlgo.Native,
                                (3, 3, 3), (1, 1, 1), (1, 1, 1), (1, 1, 1), (0, 0, 0), True, True)
    x = torch.zeros((3, 64), dtype=torch.float16)
    with pytest.raises(ValueError, match="int8 weights"):
        w8a8.linear(x, torch.zeros((5, 64)), torch.zeros(5), torch.zeros(5, dtype=torch.float16))
    with pytest.raises(ValueError, match="incompatible"):
        w8a8.linear(x, torch.zeros((5, 32), dtype=torch.int8), torch.zeros(5), torch.zeros(5, dtype=torch.float16))
    with pytest.raises(ValueError, match="divisible by 64"):
        w8a8.quantize_activation(torch.zeros((2, 72), dtype=torch.float16))


def test_sparse_tensor_validation():
    from hi3d_amd import nn as snn
    from hi3d_amd import sparse_backend

    feats = torch.zeros((2, 3))
    with pytest.raises(ValueError, match=r"\[N, 4\]"):
        sparse_backend.sparse_tensor(feats, torch.zeros((2, 3), dtype=torch.int32))
    with pytest.raises(ValueError, match="non-negative"):
        sparse_backend.sparse_tensor(feats, torch.tensor([[0, -1, 0, 0], [0, 1, 1, 1]]))
    with pytest.raises(ValueError, match="outside spatial_shape"):
        sparse_backend.sparse_tensor(feats, torch.tensor([[0, 0, 0, 0], [0, 4, 1, 1]]), (4, 4, 4))
    t = sparse_backend.sparse_tensor(feats, torch.tensor([[0, 0, 0, 0], [1, 3, 1, 2]]))
    assert t.spatial_shape == [4, 2, 3] and t.batch_size == 2
    with pytest.raises(ValueError, match="rows"):
        sparse_backend.replace_feats(t, torch.zeros((3, 3)))
    with pytest.raises(ValueError, match="cannot be empty"):
        snn.SparseTensor(torch.zeros((0, 3)), torch.zeros((0, 4), dtype=torch.int32))
    with pytest.raises(ValueError, match="contiguous"):
        snn.SparseTensor(torch.zeros((3, 2)), torch.tensor([[0, 0, 0, 0], [1, 0, 0, 1], [0, 0, 1, 0]]))


def test_product_path_refuses_host_tensors():
    """No CPU fallback: compute entry points reject host tensors loudly."""
    from hi3d_amd import kmap, kernels, w8a8

    coords = torch.zeros((1, 4), dtype=torch.int32)
    with pytest.raises(ValueError, match="ROCm GPU only"):
        kmap.build_kernel_map(coords, [2, 2, 2])
    with pytest.raises(ValueError, match="ROCm GPU only"):
        w8a8.quantize_activation(torch.zeros((2, 64), dtype=torch.float16))
    with pytest.raises(ValueError, match="ROCm GPU only"):
        kernels.layer_norm_modulate(torch.zeros((2, 8), dtype=torch.float16), 1e-6)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from hi3d_amd import _lib

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "absent.so")
    with pytest.raises(ImportError, match="build the gfx950 HIP library"):
        _lib.lib()


def test_spconv_install_registers_and_refuses_to_shadow():
    from hi3d_amd import spconv

    saved = {k: sys.modules.pop(k) for k in list(sys.modules) if k == "spconv" or k.startswith("spconv.")}
    try:
        spconv.install()
        import spconv as registered  # noqa: F401
        from spconv.pytorch import SubMConv3d
        from spconv.pytorch.core import IndiceData
        from spconv.pytorch.ops import get_indice_pairs

        assert SubMConv3d is spconv.SubMConv3d and IndiceData is spconv.IndiceData
        assert get_indice_pairs is spconv.get_indice_pairs
        spconv.install()  # idempotent
        spconv.uninstall()
        assert "spconv" not in sys.modules
        sys.modules["spconv"] = types.ModuleType("spconv")  # a "real" spconv
        with pytest.raises(RuntimeError, match="refusing to shadow"):
            spconv.install()
    finally:
        for k in [k for k in sys.modules if k == "spconv" or k.startswith("spconv.")]:
            del sys.modules[k]
        sys.modules.update(saved)


def test_workload_generators_match_stated_sizes():
    from hi3d_amd import workloads

    c1 = workloads.sphere_shell()
    assert c1.shape == (45128, 4) and c1.dtype == "int32"
    assert len(set(map(tuple, c1.tolist()))) == len(c1)
    c2 = workloads.coords_for("subm3_c128_fp16")
    assert 400_000 <= len(c2) <= 600_000
    assert c2[:, 1:].min() >= 0 and c2[:, 1:].max() < 256


def test_bench_main_calls_defined_functions():
    """Every workload function bench.py's main() calls is defined in bench.py (a CPU check
    of the driver contract's entry point; the workloads themselves need the GPU)."""
    import ast

    tree = ast.parse((ROOT / "bench.py").read_text())
    defined = {node.name for node in tree.body if isinstance(node, ast.FunctionDef)}
    main = next(node for node in tree.body if isinstance(node, ast.FunctionDef) and node.name == "main")
    called = {node.func.id for node in ast.walk(main) if isinstance(node, ast.Call) and isinstance(node.func, ast.Name)}
    wanted = {name for name in called if name.startswith(("bench_", "cpu_baseline", "measured_traffic"))}
    assert wanted and wanted <= defined, sorted(wanted - defined)


def test_res_block_state_dict_names_match_the_reference():
    """``resblock.SparseResBlock3d`` keeps the reference module's parameter names and
    shapes (src/sparc3d/models/transformers/sparc3d_transformer.py:109-129), so its state
    dict loads unchanged; the linear starts at zero (``zero_module``)."""
    from hi3d_amd.resblock import SparseResBlock3d

    m = SparseResBlock3d(256, 2112, out_channels=512)
    shapes = {k: tuple(v.shape) for k, v in m.state_dict().items()}
    assert shapes == {
        "norm1.weight": (256,), "norm1.bias": (256,),
        "conv1.conv.weight": (256, 3, 3, 3, 256), "conv1.conv.bias": (256,),
        "conv2.conv.weight": (256, 3, 3, 3, 256), "conv2.conv.bias": (256,),
        "linear.weight": (512, 256), "linear.bias": (512,),
        "emb_layers.1.weight": (512, 2112), "emb_layers.1.bias": (512,),
        "skip_connection.weight": (512, 256), "skip_connection.bias": (512,),
    }
    assert not m.linear.weight.any() and not m.linear.bias.any()
    plain = SparseResBlock3d(256, 2112)
    assert "skip_connection.weight" not in plain.state_dict() and plain.hidden_channels == 128
    assert SparseResBlock3d(64, 8, downsample=True).updown is not None
