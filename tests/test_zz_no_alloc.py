"""hx_exl3_gemm_noalloc (the allocation-free linear: its scratch is the library's fixed per-GPU
device array) through the C ABI against hx_exl3_gemm with a workspace: bit-identical outputs on two
calls in a row, the second smaller, on the GEMV and the MFMA paths; and the size limit."""
import numpy as np
import pytest

from helpers import make_linear, make_x

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import exl3
    return exl3


def _dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


@pytest.mark.parametrize("shapes", [((8, 4096, 12288, 4), (1, 4096, 2048, 2)),    # GEMV, split-K partials
                                    ((200, 2048, 1024, 3), (40, 1024, 512, 2))])  # MFMA, staged activations
def test_noalloc_equals_workspace_path(hx, shapes):
    import torch
    for i, (M, K, N, bits) in enumerate(shapes):
        tr, suh, svh = make_linear(70 + i, K, N, bits)
        x = _dev(make_x(80 + i, M, K))
        w = hx.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), hx.MUL1)
        y_ws = torch.empty((M, N), dtype=torch.float32, device="cuda")
        y_na = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
        p1 = hx.gemm(y_ws, x, w, M, N, K, bits, True)
        p2 = hx.gemm_noalloc(y_na, x, w, M, N, K, bits, True)
        torch.cuda.synchronize()
        assert p1 == p2
        assert torch.equal(y_ws, y_na), f"call {i}: M={M} K={K} N={N}"


def test_noalloc_rejects_oversize(hx):
    import torch
    from helios_glm53flash_amd._lib import HxError, lib
    cap = lib.hx_exl3_gemm_noalloc_max_bytes()
    assert cap == 8 << 20
    M, K, N = 4096, 4096, 256  # M*K fp16 = 32 MiB of staged activations
    assert lib.hx_exl3_gemm_workspace_size(M, N, K) > cap
    tr, suh, svh = make_linear(5, K, N, 2)
    w = hx.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), hx.MUL1)
    x = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    with pytest.raises(HxError, match="scratch"):
        hx.gemm_noalloc(y, x, w, M, N, K, 2, True)
