"""The C-ABI library loads without a GPU, exports every symbol include/ghost_hip.h declares,
and rejects bad arguments with an error status and message before touching the device."""
import ctypes
import re
from pathlib import Path

import pytest

from ghostsuite_amd import _native

HEADER = Path(__file__).resolve().parent.parent / "include" / "ghost_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gs_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    names = declared_functions()
    assert names, "no functions parsed from the header"
    assert set(names) == set(_native.exported_symbols())


def test_library_exports_every_declared_symbol():
    lib = _native.load_library()
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} missing from libghost_hip.so"
    assert lib.gs_abi_version() == _native.ABI_VERSION


def test_invalid_arguments_return_status_and_message():
    lib = _native.load_library()
    rc = lib.gs_linear_dot(None, None, 0, 0, 1, 0, 4, 8, 8, 0, 0, 0, None, None, None, 0, None)
    assert rc == -1
    assert b"invalid" in lib.gs_last_error()
    rc = lib.gs_linear_dot(None, None, 7, 4, 1, 3, 4, 8, 8, 0, 0, 0, None, None, None, 0, None)
    assert rc == -2  # dtype
    # well-formed request without workspace
    rc = lib.gs_linear_dot(ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 4, 1, 3, 4, 8, 8, 0, 0,
                           0, ctypes.c_void_p(16), None, None, 0, None)
    assert rc == -3
    assert b"workspace" in lib.gs_last_error()
    assert lib.gs_kron_proj(None, None, 0, 1, 1, 4, 4, None, None, 0, 40, 4, 0, 1.0, None, 1,
                            None, 0, None) == -1
    assert lib.gs_kron_proj(ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 1, 1, 4, 4,
                            ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 40, 4, 0, 1.0,
                            ctypes.c_void_p(16), 1, None, 0, None) == -3  # k = 40: needs ws
    # F = 4096 takes the wide-row path: a well-formed request that needs its workspace
    assert lib.gs_layernorm_dot(ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 4, 1, 3, 2, 4096,
                                1e-5, None, None, None, None, 1, 1.0, None, 0, None) == -3


def test_workspace_queries():
    lib = _native.load_library()
    assert lib.gs_linear_dot_workspace(0, 32, 8, 1024, 768, 3072, 0, 1, 0) > 0
    assert lib.gs_linear_dot_workspace(0, 32, 32, 1024, 768, 3072, 0, 1, 0) == 0  # no train rows
    assert lib.gs_linear_dot_workspace(0, 32, 8, 1024, 768, 3072, 1, 1, 1) == 0   # presum pairs
    assert lib.gs_embedding_dot_workspace(20, 4, 1024, 768, 50257) > 4 * 50257
    assert lib.gs_layernorm_dot_workspace(20, 1024, 768) > 0
    assert lib.gs_kron_proj_workspace(32, 1024, 16, 16) >= 32 * 16 * 16 * 16 * 4


def test_auto_algorithm_choice_is_host_only():
    lib = _native.load_library()
    # BASELINE microbench at T=1024: the val-gradient form is ~10x fewer flops
    assert lib.gs_linear_dot_algo(0, 32, 8, 1024, 768, 3072, 0, 0, 0) == _native.ALGO_VALGRAD
    # short sequences with wide layers: the ghost Gram is cheaper
    assert lib.gs_linear_dot_algo(0, 20, 4, 8, 1024, 4096, 0, 0, 0) == _native.ALGO_GHOST
    assert lib.gs_linear_dot_algo(0, 20, 4, 8, 1024, 4096, 0, 2, 0) == _native.ALGO_VALGRAD


def test_cpu_tensors_are_rejected_loudly():
    import torch
    with pytest.raises(_native.GhostHipError, match="ROCm GPU"):
        _native.HipOps().linear_dot(torch.zeros(4, 3, 8), torch.zeros(4, 3, 8), 1)


def test_noalloc_rejects_calls_beyond_its_scratch_before_touching_the_device():
    """gs_linear_dot_noalloc checks its fixed scratch size on the host: a call that needs
    more (the GPT-2 lm_head shape, 472 MiB) fails with GS_ERR_UNSUPPORTED and a message
    naming the need, before any HIP call."""
    lib = _native.load_library()
    P16 = ctypes.c_void_p(256)
    need = lib.gs_linear_dot_noalloc_bytes(P16, P16, 0, 20, 4, 1024, 768, 50257, 0, 2, 0)
    assert need > (128 << 20)
    rc = lib.gs_linear_dot_noalloc(P16, P16, 0, 20, 4, 16, 1024, 768, 50257, 0, 2, 0, P16,
                                   None, None)
    assert rc == -5
    assert b"scratch" in lib.gs_last_error() and str(need).encode() in lib.gs_last_error()
    # argument checks as gs_linear_dot's
    assert lib.gs_linear_dot_noalloc(None, None, 0, 4, 1, 3, 4, 8, 8, 0, 0, 0, None, None,
                                     None) == -1
    assert lib.gs_linear_dot_noalloc(P16, P16, 7, 4, 1, 3, 4, 8, 8, 0, 0, 0, P16, None,
                                     None) == -2
    # the GPT-2-small block layers fit
    for d_in, d_out, sem in ((768, 2304, 1), (768, 768, 1), (768, 3072, 0), (3072, 768, 0)):
        assert 0 < lib.gs_linear_dot_noalloc_bytes(P16, P16, 0, 20, 4, 1024, d_in, d_out, sem,
                                                   0, 0) <= (128 << 20)
