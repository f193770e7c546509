"""ctypes binding of the C-ABI in ``include/mintext_moe.h``.

The shared library ``mintext_amd/_lib/libmintext_moe.so`` is the only compute path of this
package: every public op enqueues HIP kernels from it on the current torch stream.  When the
library has not been built, or the tensors are not on a ROCm device, the ops raise
immediately -- there is deliberately no CPU or eager-PyTorch fallback.

PyTorch is used only as the device-memory and stream provider (``torch.empty`` for outputs
and workspaces, ``torch.cuda.current_stream()`` for the stream handle).
"""
from __future__ import annotations

import ctypes
import functools
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libmintext_moe.so"

# status codes / dtype codes / scoring modes, as in include/mintext_moe.h
MTX_OK = 0
MTX_ERR_ARG = -1
MTX_ERR_WORKSPACE = -2
MTX_ERR_UNSUPPORTED = -3
MTX_ERR_HIP = -4
MTX_F32, MTX_BF16, MTX_FP8E4M3 = 0, 1, 2
MTX_SCORING_SOFTMAX, MTX_SCORING_SIGMOID_GROUP = 0, 1
MTX_GMM_OP_FWD, MTX_GMM_OP_SWIGLU, MTX_GMM_OP_DLHS = 0, 1, 2

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float

# name -> (restype, argtypes); kept in the order of the header
SIGNATURES = {
    "mtx_status_string": (ctypes.c_char_p, [_I]),
    "mtx_last_hip_error": (_I, []),
    "mtx_version": (_I, []),
    "mtx_router_topk": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _I64, _I64, _I, _F, _P, _P, _P, _P]),
    "mtx_router_topk_shared": (_I, [_P, _I, _I64, _I64, _I64, _I, _P, _I64, _I64, _I, _F, _I64, _P, _P, _P, _P]),
    "mtx_gate_router_topk": (_I, [_P, _I, _P, _I64, _I64, _I64, _I64, _I, _P, _I64, _I64, _I, _F, _I64, _P, _P, _P,
                                   _P, _P]),
    "mtx_router_topk_bwd": (_I, [_P, _I, _I64, _I64, _I64, _I, _I, _F, _P, _I64, _P, _P, _P, _I, _P]),
    "mtx_expert_bias_update": (_I, [_P, _I64, _F, _P, _P]),
    "mtx_route_workspace_size": (_I64, [_I64, _I64, _I64]),
    "mtx_route": (_I, [_P, _I, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "mtx_gather_rows": (_I, [_P, _I, _I64, _I64, _P, _I64, _I64, _P, _P]),
    "mtx_scatter_rows": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "mtx_invert_permutation": (_I, [_P, _I64, _P, _P]),
    "mtx_unroute": (_I, [_P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I, _P]),
    "mtx_unroute_add": (_I, [_P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _I, _P, _I, _P]),
    "mtx_unroute_bwd": (_I, [_P, _I, _P, _I, _P, _P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "mtx_gmm_workspace_size": (_I64, [_I64, _I64]),
    "mtx_gmm": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_swiglu": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_dlhs": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_tgmm": (_I, [_P, _P, _P, _I, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_tiled": (_I, [_I, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_tiled_noalloc": (_I, [_I, _P, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P]),
    "mtx_gmm_gathered": (_I, [_I, _P, _I64, _P, _I64, _P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64, _P, _P, _I64,
                              _P]),
    "mtx_swiglu": (_I, [_P, _I, _I64, _I64, _P, _P]),
    "mtx_swiglu_bwd": (_I, [_P, _P, _I, _I64, _I64, _P, _P]),
    "mtx_quant_fp8_rows": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "mtx_route_quant_fp8": (_I, [_P, _I, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64, _P]),
    "mtx_quant_fp8_weights": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "mtx_gmm_fp8": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_fp8_swiglu": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "mtx_gmm_fp8_swiglu_gathered": (_I, [_P, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P,
                                         _P, _I64, _P]),
    "mtx_quant_fp8_rows_p2": (_I, [_P, _I, _I64, _I64, _P, _P, _P]),
    "mtx_quant_fp8_weights_p2": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "mtx_gmm_fp8_p2": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_gmm_fp8_swiglu_p2": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _I64, _P]),
    "mtx_gmm_fp8_swiglu_gathered_p2": (_I, [_P, _P, _I64, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _P,
                                            _P, _I64, _P]),
    "mtx_quant_fp8_weights_t": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "mtx_gmm_fp8_dlhs": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_fp8_grouped_chunks": (_I64, [_I64, _I64]),
    "mtx_fp8_grouped_workspace_size": (_I64, [_I64]),
    "mtx_quant_fp8_grouped_t": (_I, [_P, _I, _P, _I64, _I64, _I64, _I, _P, _P, _P, _I64, _P]),
    "mtx_tgmm_fp8": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_quant_fp8_weights_t_p2": (_I, [_P, _I, _I64, _I64, _I64, _P, _P, _P]),
    "mtx_gmm_fp8_dlhs_p2": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_quant_fp8_grouped_t_p2": (_I, [_P, _I, _P, _I64, _I64, _I64, _I, _P, _P, _P, _I64, _P]),
    "mtx_tgmm_fp8_p2": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _P, _P, _I64, _P]),
    "mtx_transpose_batched": (_I, [_P, _I, _I64, _I64, _I64, _I64, _I64, _P, _I64, _I64, _P]),
    "mtx_stream_copy": (_I, [_P, _P, _I64, _I, _I64, _P]),
}


class MtxError(RuntimeError):
    """A C-ABI entry point returned a non-zero status."""

    def __init__(self, name: str, status: int, detail: str = ""):
        self.status = status
        super().__init__(f"{name} failed: {detail or status}")


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"MI355X kernel library not found at {LIB_PATH}; build it with "
            "`python -m mintext_amd.build` (there is no fallback path)")
    handle = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def call(name: str, *args) -> None:
    """Invoke ``name`` and raise MtxError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != MTX_OK:
        detail = lib().mtx_status_string(rc).decode()
        if rc == MTX_ERR_HIP:
            detail += f" (hipError {lib().mtx_last_hip_error()})"
        raise MtxError(name, rc, detail)


def query(name: str, *args) -> int:
    v = getattr(lib(), name)(*args)
    if v < 0:
        raise MtxError(name, int(v), "invalid sizes")
    return int(v)


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return MTX_F32
    if dt == torch.bfloat16:
        return MTX_BF16
    if dt == torch.float8_e4m3fn or dt == torch.uint8:
        return MTX_FP8E4M3
    raise TypeError(f"unsupported dtype {dt}; expected float32, bfloat16 or float8_e4m3fn")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "mintext_amd ops run only on a ROCm GPU tensor (got a CPU tensor); "
                "there is no CPU fallback")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def exported_symbols() -> list[str]:
    """Names of SIGNATURES that the built library actually exports."""
    handle = ctypes.CDLL(str(LIB_PATH))
    return [n for n in SIGNATURES if hasattr(handle, n)]
