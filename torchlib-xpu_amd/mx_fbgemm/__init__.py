"""mx_fbgemm: MI355X (gfx950) implementations of fbgemm_gpu's jagged and
table-batched-embedding operators, registered under ``torch.ops.fbgemm``.

``import mx_fbgemm`` loads the native extension, whose static initializers
define the ``fbgemm`` schemas and register the GPU implementations -- the
same plugin shape as the reference's loader
(reference: packages/torchcodec-xpu/src/torchcodec_xpu/__init__.py:25-56):
load at import, and on failure raise one RuntimeError that says which
library failed and why.

There is no CPU fallback: the operators accept HIP tensors only, and the
import fails loudly when the native libraries are missing.
"""

from __future__ import annotations

import ctypes
import traceback
from pathlib import Path

import torch

__version__ = "0.1.0"

_LIB_DIR = Path(__file__).resolve().parent / "lib"
KERNEL_LIBRARY = _LIB_DIR / "libmx_fbgemm_kernels.so"
OPS_LIBRARY = _LIB_DIR / "mx_fbgemm_ops.so"

# Ops this package defines in the ``fbgemm`` namespace.
OPS = (
    "jagged_to_padded_dense_forward",
    "jagged_to_padded_dense",
    "jagged_to_padded_dense_backward",
    "dense_to_jagged_forward",
    "dense_to_jagged",
    "jagged_dense_elementwise_add_jagged_output",
    "split_embedding_codegen_forward_unweighted_cuda",
    "split_embedding_codegen_forward_weighted_cuda",
    "get_infos_metadata",
    "transpose_embedding_input",
    "split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_cuda",
    "split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_cuda",
    "split_embedding_codegen_grad_indice_weights_cuda",
    "generate_vbe_metadata",
    "split_embedding_codegen_forward_unweighted_vbe_cuda",
    "split_embedding_codegen_forward_weighted_vbe_cuda",
    "split_embedding_backward_codegen_rowwise_adagrad_unweighted_exact_vbe_cuda",
    "split_embedding_backward_codegen_rowwise_adagrad_weighted_exact_vbe_cuda",
    "split_embedding_codegen_grad_indice_weights_vbe_cuda",
    "split_embedding_codegen_lookup_rowwise_adagrad_function",
    "int_nbit_split_embedding_codegen_lookup_function",
    "bounds_check_indices",
    "FloatToFused8BitRowwiseQuantized",
    "HalfToFused8BitRowwiseQuantized",
    "FloatOrHalfToFused8BitRowwiseQuantized",
    "Fused8BitRowwiseQuantizedToFloat",
    "Fused8BitRowwiseQuantizedToHalf",
    "FloatToFusedNBitRowwiseQuantizedSBHalf",
    "HalfToFusedNBitRowwiseQuantizedSBHalf",
    "FloatOrHalfToFusedNBitRowwiseQuantizedSBHalf",
    "FusedNBitRowwiseQuantizedSBHalfToFloat",
    "FusedNBitRowwiseQuantizedSBHalfToHalf",
)

_loaded = False


def _fbgemm_already_defined() -> list[str]:
    """Names of our ops that some other library already defined."""
    found = []
    for name in OPS:
        try:
            torch._C._dispatch_find_schema_or_throw(f"fbgemm::{name}", "")
            found.append(name)
        except RuntimeError:
            pass
    return found


def load_mx_fbgemm_library() -> None:
    """Load the kernel library and the torch extension (idempotent)."""
    global _loaded
    if _loaded:
        return
    clash = _fbgemm_already_defined()
    if clash:
        raise RuntimeError(
            "torch.ops.fbgemm already defines " + ", ".join(clash) + ": another FBGEMM "
            "implementation (e.g. fbgemm_gpu) is loaded in this process. mx_fbgemm replaces "
            "it and cannot be loaded alongside it."
        )
    # Step 1: the kernel library, loaded global so that the extension's
    # DT_NEEDED entry resolves to this exact file.  Step 2: the extension,
    # whose static initializers register the ops.
    steps = (
        ("kernel library", KERNEL_LIBRARY,
         lambda: ctypes.CDLL(str(KERNEL_LIBRARY), mode=ctypes.RTLD_GLOBAL)),
        ("torch extension", OPS_LIBRARY, lambda: torch.ops.load_library(str(OPS_LIBRARY))),
    )
    for what, path, load in steps:
        if not path.is_file():
            raise RuntimeError(
                f"Could not load mx_fbgemm: its {what} {path} does not exist. Build it with "
                "`python torchlib-xpu_amd/mx_fbgemm/_build.py` (or __graft_entry__.build()); "
                "the operators have no CPU implementation to fall back on."
            )
        try:
            load()
        except Exception as exc:
            raise RuntimeError(
                f"Could not load mx_fbgemm: loading its {what} {path} failed with "
                f"{type(exc).__name__}: {exc}\n"
                f"This process runs torch {torch.__version__} with HIP {torch.version.hip}; "
                "an extension built against another torch, or a ROCm runtime "
                "(libamdhip64) missing from the loader path, fails this way. Rebuild with "
                "`python torchlib-xpu_amd/mx_fbgemm/_build.py`.\n"
                + "".join(traceback.format_exception(type(exc), exc, exc.__traceback__))
            ) from exc
    _loaded = True


load_mx_fbgemm_library()

from .sparse_types import (  # noqa: E402
    BoundsCheckMode,
    ComputeDevice,
    EmbeddingLocation,
    EmbOptimType,
    PoolingMode,
    SparseType,
)

__all__ = [
    "BoundsCheckMode",
    "ComputeDevice",
    "EmbeddingLocation",
    "EmbOptimType",
    "PoolingMode",
    "SparseType",
    "KERNEL_LIBRARY",
    "OPS_LIBRARY",
    "load_mx_fbgemm_library",
]
