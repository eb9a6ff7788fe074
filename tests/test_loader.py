"""The package loader: it fails loudly (one RuntimeError naming the library
that is missing or failed to load) when the native libraries are absent or
broken, as the reference's loader fails at import
(packages/torchcodec-xpu/src/torchcodec_xpu/__init__.py:33-54); and the ops it
registers have no CPU kernels (no silent CPU fallback)."""

import shutil
import subprocess
import sys
from pathlib import Path

import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
PKG = REPO / "torchlib-xpu_amd" / "mx_fbgemm"


def test_missing_library_raises(tmp_path):
    dst = tmp_path / "mx_fbgemm"
    dst.mkdir()
    for f in PKG.glob("*.py"):
        shutil.copy(f, dst / f.name)  # no lib/ directory
    code = ("import sys; sys.path.insert(0, %r)\n"
            "try:\n    import mx_fbgemm\nexcept RuntimeError as e:\n"
            "    print('RAISED:' + str(e).splitlines()[0])\n" % str(tmp_path))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert "RAISED:Could not load mx_fbgemm: its kernel library" in out.stdout, \
        out.stdout + out.stderr
    assert "does not exist" in out.stdout


def test_unloadable_library_raises(tmp_path):
    """A kernel library that is present but cannot be loaded (here: not an ELF
    file) is reported with the loader's own error, not swallowed."""
    dst = tmp_path / "mx_fbgemm"
    (dst / "lib").mkdir(parents=True)
    for f in PKG.glob("*.py"):
        shutil.copy(f, dst / f.name)
    (dst / "lib" / "libmx_fbgemm_kernels.so").write_bytes(b"not a shared object")
    code = ("import sys; sys.path.insert(0, %r)\n"
            "try:\n    import mx_fbgemm\nexcept RuntimeError as e:\n"
            "    print('RAISED:' + str(e).splitlines()[0])\n" % str(tmp_path))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert "RAISED:Could not load mx_fbgemm: loading its kernel library" in out.stdout, \
        out.stdout + out.stderr
    assert "OSError" in out.stdout


def test_cpu_tensors_have_no_kernel():
    import mx_fbgemm  # noqa: F401

    off = torch.tensor([0, 2, 3])
    vals = torch.randn(3, 4)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.fbgemm.jagged_to_padded_dense_forward(vals, [off], [2], 0.0)
    with pytest.raises((NotImplementedError, RuntimeError)):
        torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function(
            torch.zeros(10, dtype=torch.uint8), torch.zeros(0, dtype=torch.uint8),
            torch.zeros(1, dtype=torch.int32), torch.zeros(1, dtype=torch.int64),
            torch.zeros(1, dtype=torch.uint8), torch.tensor([0, 8], dtype=torch.int32), 8,
            0, 0, 8, 0, 0, torch.zeros(1, dtype=torch.int32), torch.tensor([0, 1], dtype=torch.int32),
            0, None, 1, None, None, 16)


def test_schemas_registered():
    import mx_fbgemm

    for name in mx_fbgemm.OPS:
        assert hasattr(torch.ops.fbgemm, name), name
    s = str(torch.ops.fbgemm.int_nbit_split_embedding_codegen_lookup_function.default._schema)
    assert "int? row_alignment=None" in s and "Tensor weights_tys" in s
