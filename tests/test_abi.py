"""The C-ABI library loads and exports every entry point that include/mintext_moe.h declares,
with the argument counts of the Python binding; host-side validation rejects bad arguments
before any GPU work (these calls return before touching the device, so they run on CPU)."""
from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT
from mintext_amd import _lib

HEADER = ROOT / "include" / "mintext_moe.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(mtx_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else args.count(",") + 1
        decls[m.group(1)] = n
    return decls


@pytest.fixture(scope="module")
def built():
    if not _lib.LIB_PATH.exists():
        from mintext_amd import build

        build.build(verbose=False)
    return _lib.lib()


def test_header_matches_binding():
    decls = _declared()
    assert set(decls) == set(_lib.SIGNATURES), set(decls) ^ set(_lib.SIGNATURES)
    for name, n in decls.items():
        assert len(_lib.SIGNATURES[name][1]) == n, name


def test_library_exports_all_symbols(built):
    handle = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in _declared() if not hasattr(handle, n)]
    assert not missing, missing


def test_status_strings(built):
    assert built.mtx_status_string(0) == b"ok"
    assert b"workspace" in built.mtx_status_string(-2)
    assert built.mtx_version() >= 1


def test_workspace_queries(built):
    assert built.mtx_route_workspace_size(8192, 2, 8) > 0
    assert built.mtx_route_workspace_size(-1, 2, 8) < 0
    a = built.mtx_gmm_workspace_size(16384, 8)
    b = built.mtx_gmm_workspace_size(131072, 128)
    assert 0 < a < b


def test_host_validation_rejects_bad_args(built):
    # every call below must return before any HIP API call (no device here)
    P = None
    assert built.mtx_route(P, 1, P, 4, 8, 2, 0, P, P, P, P, P, P, P, 0, P) == _lib.MTX_ERR_ARG  # E = 0
    assert built.mtx_route(P, 7, P, 4, 8, 2, 4, P, P, P, P, P, P, P, 0, P) == _lib.MTX_ERR_ARG  # dtype
    ws = ctypes.create_string_buffer(16)
    dummy = ctypes.addressof(ws)
    assert built.mtx_route(P, 1, dummy, 4, 8, 2, 4, P, dummy, dummy, P, P, P, dummy, 8, P) == \
        _lib.MTX_ERR_WORKSPACE
    assert built.mtx_router_topk(P, 1, 4, 8, 9, 0, P, 1, 1, 1, 1.0, P, P, P, P) == _lib.MTX_ERR_ARG  # K > E
    assert built.mtx_router_topk(P, 1, 4, 10, 2, 1, P, 3, 1, 1, 1.0, P, P, P, P) == _lib.MTX_ERR_ARG  # E % groups
    assert built.mtx_gmm(P, P, P, 0, 16, 8, 4, 2, P, P, 0, P) == _lib.MTX_ERR_WORKSPACE
    assert built.mtx_gmm(P, P, P, 5, 16, 8, 4, 2, P, P, 0, P) == _lib.MTX_ERR_ARG  # dtype
    assert built.mtx_tgmm(P, P, P, 0, 16, 8, 4, 0, P, P, 0, P) == _lib.MTX_ERR_ARG  # E = 0
    assert built.mtx_quant_fp8_rows(P, 1, 4, 100, P, P, P) == _lib.MTX_ERR_ARG  # D % 128
    assert built.mtx_quant_fp8_weights(P, 1, 2, 128, 100, P, P, P) == _lib.MTX_ERR_ARG
    assert built.mtx_unroute(P, 1, P, P, 0, 4, 0, 8, P, 0, P) == _lib.MTX_ERR_ARG  # K = 0
    assert built.mtx_swiglu(P, 3, 4, 4, P, P) == _lib.MTX_ERR_ARG
    gw = ctypes.create_string_buffer(1 << 16)
    g = ctypes.addressof(gw)
    # gathered GEMMs: no row index, a bad index divisor, a bad tile shape, the dlhs op
    assert built.mtx_gmm_gathered(1, g, 4, P, 2, g, g, 1, 8, 64, 128, 2, 0, 0, g, g, 1 << 16, P) == _lib.MTX_ERR_ARG
    assert built.mtx_gmm_gathered(1, g, 4, g, 0, g, g, 1, 8, 64, 128, 2, 0, 0, g, g, 1 << 16, P) == _lib.MTX_ERR_ARG
    assert built.mtx_gmm_gathered(1, g, 4, g, 2, g, g, 1, 8, 64, 128, 2, 64, 0, g, g, 1 << 16, P) == _lib.MTX_ERR_ARG
    assert built.mtx_gmm_gathered(2, g, 4, g, 2, g, g, 1, 8, 64, 128, 2, 0, 0, g, g, 1 << 16, P) == _lib.MTX_ERR_ARG
    assert built.mtx_gmm_fp8_swiglu_gathered(g, g, 4, P, 2, g, g, g, 8, 256, 128, 2, g, g, P, g, 1 << 16, P) == \
        _lib.MTX_ERR_ARG


def test_gathered_swiglu_supported_predicate():
    """The host-side mirror of the gathered GEMM's shape conditions (bf16, K_in % 64, I % 128)."""
    import torch

    from mintext_amd.kernels.grouped_matmul import gathered_swiglu_supported

    x = torch.zeros(16, 256, dtype=torch.bfloat16)
    assert gathered_swiglu_supported(x, torch.zeros(4, 256, 256, dtype=torch.bfloat16))
    assert not gathered_swiglu_supported(x.float(), torch.zeros(4, 256, 256))  # f32
    assert not gathered_swiglu_supported(x, torch.zeros(4, 256, 128, dtype=torch.bfloat16))  # I = 64
    assert not gathered_swiglu_supported(x[:, :96].contiguous(), torch.zeros(4, 96, 256, dtype=torch.bfloat16))
    assert not gathered_swiglu_supported(x[:, :128], torch.zeros(4, 128, 256, dtype=torch.bfloat16))  # strided view


def test_product_refuses_cpu_tensors():
    import torch

    from mintext_amd.kernels import route

    with pytest.raises(RuntimeError, match="no CPU fallback"):
        route(torch.zeros(4, 8), torch.zeros(4, 2, dtype=torch.int32), 4)
