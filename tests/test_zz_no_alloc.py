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


_CAPTURE_SCRIPT = r"""
import sys
import numpy as np
import torch
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/tests")
from helios_glm53flash_amd import exl3
from helpers import make_linear, make_x
M, K, N, bits = 1, 4096, 2048, 2
tr, suh, svh = make_linear(90, K, N, bits)
dev = lambda a, dt=None: (torch.from_numpy(np.ascontiguousarray(a)).view(dt) if dt else torch.from_numpy(np.ascontiguousarray(a))).cuda()
w = exl3.GroupWords(dev(tr, torch.int16), dev(suh), dev(svh), exl3.MUL1)
x = dev(make_x(91, M, K))
y_g = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.graph(g, stream=s):
    # the process's first no-alloc call: the per-device scratch lookup happens inside the capture
    exl3.gemm_noalloc(y_g, x, w, M, N, K, bits, True, stream=s)
y_ws = torch.empty((M, N), dtype=torch.float32, device="cuda")
exl3.gemm(y_ws, x, w, M, N, K, bits, True)
torch.cuda.synchronize()
for rep in range(3):
    y_g.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(y_g, y_ws), rep
    exl3.gemm(y_ws, x, w, M, N, K, bits, True)  # eager work between replays
    torch.cuda.synchronize()
print("ok")
"""


def test_noalloc_first_call_under_graph_capture(hx, tmp_path):
    """The first no-alloc call of a fresh process made inside a HIP graph capture (the per-device
    scratch lookup then runs while the stream captures); three replays, with eager calls between
    them, equal the workspace path bit for bit."""
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    script = tmp_path / "capture.py"
    script.write_text(_CAPTURE_SCRIPT)
    r = subprocess.run([sys.executable, str(script), str(root)], capture_output=True, text=True, timeout=240)
    assert r.returncode == 0 and "ok" in r.stdout, (r.stdout[-1500:], r.stderr[-3000:])
