"""mx_fbgemm: MI355X (gfx950) implementations of fbgemm_gpu's jagged and
table-batched-embedding operators, registered under ``torch.ops.fbgemm``.

``import mx_fbgemm`` loads the native extension, whose static initializers
define the ``fbgemm`` schemas and register the GPU implementations -- the
same plugin shape as the reference's loader
(reference: packages/torchcodec-xpu/src/torchcodec_xpu/__init__.py:25-56):
load at import, and on failure raise one RuntimeError that lists the likely
causes and every captured traceback.

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
    exceptions = []
    try:
        # Kernel library first (global so the extension's DT_NEEDED resolves to
        # this exact file), then the extension that registers the ops.
        ctypes.CDLL(str(KERNEL_LIBRARY), mode=ctypes.RTLD_GLOBAL)
        torch.ops.load_library(str(OPS_LIBRARY))
        _loaded = True
        return
    except Exception:
        exceptions.append(traceback.format_exc())

    traceback_info = (
        "\n[start of mx_fbgemm loading traceback]\n"
        + "\n".join(exceptions)
        + "\n[end of mx_fbgemm loading traceback]."
    )
    raise RuntimeError(
        f"""Could not load mx_fbgemm. Likely causes:
          1. The native libraries were not built: run
             `python torchlib-xpu_amd/mx_fbgemm/_build.py` (or __graft_entry__.build()).
             Expected {KERNEL_LIBRARY} and {OPS_LIBRARY}.
          2. The PyTorch version ({torch.__version__}, HIP {torch.version.hip}) differs
             from the one the extension was built against.
          3. The ROCm runtime (libamdhip64) could not be found.
        The following exceptions were raised as we tried to load mx_fbgemm:
        """
        f"{traceback_info}"
    )


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
