"""smx_weight_matmul_noalloc: the allocation-free variant of smx_weight_matmul (activation parts
in a fixed per-GPU device array) gives the same outputs as smx_weight_matmul, call after call,
through the C-ABI."""
import ctypes

import numpy as np
import pytest

import oracle as O
from tests.helpers import quantized

pytestmark = pytest.mark.gpu


def _fn(lib, name):
    f = getattr(lib, name)
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                  ctypes.c_void_p]
    return f


def _run(f, w, x, m, k, n, y):
    import torch
    torch.cuda.synchronize()
    rc = f(w._h, ctypes.c_void_p(x.data_ptr()), ctypes.c_void_p(y.data_ptr()), m, k, n, None)
    torch.cuda.synchronize()
    return rc


def test_noalloc_matmul_equals_matmul_on_consecutive_calls(gpu):
    import torch

    from smallmind_amd._lib import load
    from smallmind_amd.quantization import GpuWeightTensor
    lib = load()
    ref_f, na_f = _fn(lib, "smx_weight_matmul"), _fn(lib, "smx_weight_matmul_noalloc")
    # (type, n, k, m): the second call is smaller than the first (fewer rows, shorter k); then the
    # GEMV path (m < 4), a third matrix-core call, and two one-token-tile calls (the second smaller)
    cases = [(O.Q4_K, 512, 4096, 64), (O.Q8_0, 96, 2048, 20), (O.Q6_K, 256, 1024, 2), (O.Q5_K, 64, 512, 33),
             # one token tile on K-quant rows, the second call smaller
             (O.Q5_K, 2048, 2048, 16), (O.Q4_K, 300, 1024, 8)]
    for i, (qt, n, k, m) in enumerate(cases):
        w = GpuWeightTensor(qt, n, k, quantized(qt, (n, k), seed=50 + i))
        x = torch.randn(m, k, device="cuda", generator=torch.Generator("cuda").manual_seed(i))
        y_ref = torch.full((m, n), float("nan"), device="cuda")
        y_na = torch.full((m, n), float("nan"), device="cuda")
        assert _run(ref_f, w, x, m, k, n, y_ref) == 0
        assert _run(na_f, w, x, m, k, n, y_na) == 0, lib.smx_last_error()
        assert torch.equal(y_ref, y_na), (i, float((y_ref - y_na).abs().max()))
        # and against the oracle's float64 GEMV of the same blocks (the GEMM's 2e-5 bound)
        blocks = quantized(qt, (n, k), seed=50 + i)
        xr = x.cpu().numpy()
        for r in (0, m - 1):
            ref = O.gemv_f64(qt, blocks, n, k, xr[r])
            err = np.abs(y_na[r].cpu().numpy() - ref).max() / np.abs(ref).max()
            assert err < 2e-5, (i, r, err)
        w.close()


def test_noalloc_matmul_rejects_sizes_beyond_its_scratch(gpu):
    import torch

    from smallmind_amd._lib import load
    from smallmind_amd.quantization import GpuWeightTensor
    lib = load()
    na_f = _fn(lib, "smx_weight_matmul_noalloc")
    n, k, m = 32, 8192, 16 * 65   # 65 token tiles x 256 sub-blocks x 3 KB > 16 MiB
    w = GpuWeightTensor(O.Q8_0, n, k, quantized(O.Q8_0, (n, k), seed=3))
    x = torch.zeros(m, k, device="cuda")
    y = torch.zeros(m, n, device="cuda")
    assert _run(na_f, w, x, m, k, n, y) == -1
    assert b"limit" in lib.smx_last_error()
    w.close()
