"""ctypes binding of the gfx950 C ABI (``include/sparse_prefill.h``).

The shared library is built in-tree by ``python -m exp3_amd.build``. There is no
fallback: every public wrapper raises if the library is missing or a tensor is
not on a ROCm GPU.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "_C" / "libexp3_amd.so"

SPX_OK = 0
SPX_EINVAL = -1
SPX_EUNSUPPORTED = -2
SPX_ELAUNCH = -3
ABI_VERSION = 8
# int32 counters behind the attention entry points' work_queue (SPX_WORK_QUEUE_INTS)
WORK_QUEUE_INTS = 16

SELECTOR_IDS = {"mean_balanced": 0, "cgf_mean": 1, "dispersion_mean": 2}

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float
_S = ctypes.POINTER(ctypes.c_int64)

# name -> argument types (restype is int for all compute entry points)
_PROTOTYPES = {
    "spx_block_mean_k": [_P, _S, _I, _I, _I, _I, _I, _P, _P],
    "spx_block_descriptors": [_P, _S, _P, _S, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P],
    "spx_block_pool": [_P, _S, _P, _S, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P],
    "spx_v1_scores": [_P, _S, _P, _S, _I, _I, _I, _I, _I, _I, _F, _P, _S, _P],
    "spx_deal_output_score": [_P, _S, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _P, _P, _P],
    "spx_protected_selection": [_P, _S, _I, _I, _I, _I, _F, _I, _I, _I, _P, _P, _P, _P],
    "spx_v1_route": [_P, _S, _P, _S, _I, _I, _I, _I, _I, _I, _F, _F, _I, _I, _I, _P, _P, _P,
                     _P, _P],
    "spx_indices_from_mask": [_P, _I, _I, _I, _I, _P, _P, _P],
    "spx_mask_from_indices": [_P, _P, _I, _I, _I, _I, _P, _P],
    "spx_selector_scores": [_P, _S, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P, _P, _S,
                            _P],
    "spx_selector_scores_noalloc": [_P, _S, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _F, _P,
                                    _S, _P],
    "spx_exact_attention": [_P, _S, _P, _P, _P, _S, _P, _S, _I, _I, _I, _I, _I, _I, _F, _P,
                            _S, _P, _S, _P, _P],
    "spx_sparse_attention_mean": [_P, _S, _P, _P, _P, _S, _P, _S, _P, _P, _P, _I, _I, _I, _I,
                                  _I, _I, _F, _P, _S, _P, _S, _P, _P],
    "spx_mean_tail": [_P, _S, _P, _S, _P, _S, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _S, _P,
                      _S, _P],
    "spx_merge_exact_mean": [_P, _S, _P, _S, _P, _S, _P, _S, _I, _I, _I, _I, _P, _S, _P, _S, _P],
    "spx_selection_accounting": [_P, _I, _I, _I, _I, _I, _I, _P, _P],
    "spx_tile_mean_query": [_P, _S, _I, _I, _I, _I, _I, _P, _P],
    "spx_rescue_choice": [_P, _P, _I, _I, _I, _I, _I, _I, _P, _P],
    "spx_rescue_tail": [_P, _S, _P, _P, _P, _S, _P, _S, _P, _P, _S, _P, _P, _I, _I, _I, _I, _I,
                        _I, _I, _F, _P, _S, _P, _S, _P],
    "spx_sparse_attention_rescue": [_P, _S, _P, _P, _P, _S, _P, _S, _P, _P, _S, _P, _P, _I, _I,
                                    _I, _I, _I, _I, _I, _F, _P, _S, _P, _S, _P, _P],
}

# helpers with other return types
_SIZE_FUNCTIONS = {"spx_selector_workspace_bytes": [_I, _I, _I, _I]}

EXPORTED_SYMBOLS = tuple(_PROTOTYPES) + tuple(_SIZE_FUNCTIONS) + ("spx_last_error",
                                                                   "spx_abi_version")

_lib = None


def load() -> ctypes.CDLL:
    """Load the HIP library once (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY_PATH.exists():
        raise RuntimeError(
            f"exp3_amd HIP library not found at {LIBRARY_PATH}; build it with "
            "`python -m exp3_amd.build` (hipcc, gfx950)")
    lib = ctypes.CDLL(str(LIBRARY_PATH))
    lib.spx_last_error.restype = ctypes.c_char_p
    lib.spx_last_error.argtypes = []
    lib.spx_abi_version.restype = ctypes.c_int
    lib.spx_abi_version.argtypes = []
    for name, argtypes in _PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    for name, argtypes in _SIZE_FUNCTIONS.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int64
    if lib.spx_abi_version() != ABI_VERSION:
        raise RuntimeError(f"exp3_amd ABI mismatch: library {lib.spx_abi_version()}, "
                           f"bindings {ABI_VERSION}; rebuild the library")
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Invoke an entry point and turn a negative status into an exception."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status == SPX_OK:
        return
    message = (lib.spx_last_error() or b"").decode(errors="replace")
    if status in (SPX_EINVAL, SPX_EUNSUPPORTED):
        raise ValueError(f"{name}: {message}")
    raise RuntimeError(f"{name} failed ({status}): {message}")


# ------------------------------------------------------------ argument helpers

def ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if tensor is None else tensor.data_ptr())


def strides(tensor: torch.Tensor | None):
    if tensor is None:
        return None
    values = tensor.stride()
    return (ctypes.c_int64 * len(values))(*values)


def stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors must live on one ROCm GPU; there is no CPU path."""
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(
                "exp3_amd kernels run only on a ROCm GPU (MI355X); got a tensor on "
                f"{t.device}")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    return device


def kernel_view(x: torch.Tensor) -> torch.Tensor:
    """A [B, S, H, D] bf16 view the kernels accept (unit dim stride, 16-byte
    aligned rows); copies only when the given layout does not qualify."""
    if x.dtype != torch.bfloat16:
        raise ValueError(f"expected a bfloat16 tensor, got {x.dtype}")
    if x.dim() != 4:
        raise ValueError(f"expected a [batch, sequence, heads, dim] tensor, got {tuple(x.shape)}")
    st = x.stride()
    if st[3] == 1 and all(s % 8 == 0 for s in st[:3]) and x.data_ptr() % 16 == 0:
        return x
    return x.contiguous()
