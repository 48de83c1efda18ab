"""The reference-signature C++ layer (include/helios/exl3_compat.hpp) at run time: the C++ driver
tests/cpp/compat_driver calls helios::exl3::gemm, helios::aux::routing_ds3_nogroup,
helios::glue::moe_permute, helios::exl3::moe_grouped, helios::glue::moe_reduce_sorted,
helios::glue::gather_rows / scatter_add_rows and helios::exl3::moe_layer on the GPU, in the order
of the reference engine's call sites, and dumps inputs and outputs; this test checks them against
the CPU oracle and reads the driver's host cost per call."""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from helpers import assert_close

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
DRIVER = ROOT / "tests" / "cpp" / "compat_driver"


@pytest.fixture(scope="module")
def run(tmp_path_factory):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not DRIVER.exists():
        pytest.fail(f"{DRIVER} is not built (python -m helios_glm53flash_amd.build)")
    out = tmp_path_factory.mktemp("compat")
    r = subprocess.run([str(DRIVER), str(out)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    timing = json.loads(r.stdout.strip().splitlines()[-1])

    def load(name, dtype):
        return np.fromfile(out / f"{name}.bin", dtype=dtype)
    return load, timing


def _lin(load, p):
    return load(f"{p}_trellis", np.uint16), load(f"{p}_suh", np.uint16), load(f"{p}_svh", np.uint16)


def test_compat_gemm(run):
    from oracle import oracle as O
    load, _ = run
    K, N, bits = 1024, 512, 3
    tr, suh, svh = _lin(load, "lin")
    tr = tr.reshape(K // 16, N // 16, 16 * bits)
    for M, path in ((1, 90), (32, 1)):
        x = load(f"gemm_m{M}_x", np.uint16).reshape(M, K)
        y = load(f"gemm_m{M}_y", np.float32).reshape(M, N)
        assert int(load(f"gemm_m{M}_path", np.int32)[0]) == path
        assert_close(y, O.linear(x, tr, suh, svh, K, N, bits, 2), what=f"compat gemm M={M}")


def test_compat_had_r_128(run):
    """helios::exl3::had_r_128(..., DType::Half, 1.0f, s) as the reference's test calls it
    (test_reconstruct.cpp:330): the transform scaled by 1/sqrt(128), here with a post scale; pre and
    post together are refused."""
    from oracle import oracle as O
    load, _ = run
    x = load("had_x", np.uint16).reshape(8, 256)
    post = load("had_post", np.uint16)
    got = load("had_y", np.uint16).view(np.float16).astype(np.float64)
    ref = O.had_r_128_f16(x, None, post, 0.088388347648).view(np.float16).astype(np.float64).reshape(-1)
    assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) * 1.01)
    assert int(load("had_refused", np.int32)[0]) == 1


def test_compat_two_streams(run):
    """Config-1 linears issued on two streams at once, 20 times: both equal the single-stream result
    bit for bit (each stream has its own split-K counters)."""
    load, _ = run
    assert int(load("two_streams_same", np.int32)[0]) == 1


def _experts(load, E, hidden, inter, bits):
    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
    out = {"trellis": [[], [], []], "suh": [[], [], []], "svh": [[], [], []],
           "bits": [np.full(E, bits, np.int32) for _ in range(3)]}
    for e in range(E):
        for q, (K, N) in enumerate(shapes):
            tr, suh, svh = _lin(load, f"ex{e}_{q}")
            out["trellis"][q].append(tr.reshape(K // 16, N // 16, 16 * bits))
            out["suh"][q].append(suh)
            out["svh"][q].append(svh)
    return out


@pytest.mark.parametrize("T", [3, 20])
def test_compat_moe_sequence(run, T):
    """router -> permutation -> moe_grouped (sorted contributions) -> ordered reduction, for the
    few-token (T = 3) and the grouped prefill (T = 20) paths; then gather_rows / scatter_add_rows on
    expert 0's rows."""
    from oracle import oracle as O
    load, _ = run
    E, hidden, inter, topk, bits = 16, 512, 256, 4, 2
    tag = f"moe_t{T}"
    x = load(f"{tag}_x", np.uint16).reshape(T, hidden)
    sc = load(f"{tag}_scores", np.uint16).reshape(T, E)
    idx = load(f"{tag}_idx", np.int64).reshape(T, topk)
    w = load(f"{tag}_w", np.uint16).reshape(T, topk)
    ri, rw = O.routing(sc, topk, 2.5)
    assert np.array_equal(idx, ri)
    assert np.abs(w.view(np.float16).astype(np.float64) - rw.view(np.float16).astype(np.float64)).max() <= 2 ** -9 * 2.5
    y = load(f"{tag}_y", np.float32).reshape(T, hidden)
    ref, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), _experts(load, E, hidden, inter, bits), None, 10.0)
    assert_close(y, ref, what=f"compat moe T={T}")

    n0 = int(load(f"{tag}_n0", np.int32)[0])
    ts = load(f"{tag}_ts", np.int64)
    wsr = load(f"{tag}_wsorted", np.uint16).view(np.float16)
    contrib = load(f"{tag}_contrib", np.float32).reshape(T * topk, hidden)
    assert np.array_equal(load(f"{tag}_gather", np.uint16).reshape(n0, hidden), x[ts[:n0]])
    want = np.zeros((T, hidden), np.float32)
    want[ts[:n0]] = want[ts[:n0]] + wsr[:n0].astype(np.float32)[:, None] * contrib[:n0]
    assert np.array_equal(load(f"{tag}_scatter", np.float32).reshape(T, hidden), want)


def test_compat_moe_layer(run):
    """helios::exl3::moe_layer (hx_moe_layer) with a shared expert, 1 token."""
    from oracle import oracle as O
    load, _ = run
    E, hidden, inter, topk, bits = 16, 512, 256, 4, 2
    x = load("layer_x", np.uint16).reshape(1, hidden)
    sc = load("layer_scores", np.uint16).reshape(1, E)
    idx, w = O.routing(sc, topk, 2.5)
    sh = {"trellis": [], "suh": [], "svh": [], "bits": [bits] * 3}
    for q, (K, N) in enumerate([(hidden, inter), (hidden, inter), (inter, hidden)]):
        tr, suh, svh = _lin(load, f"sh{q}")
        sh["trellis"].append(tr.reshape(K // 16, N // 16, 16 * bits))
        sh["suh"].append(suh)
        sh["svh"].append(svh)
    yr, yo = O.moe_rows(x, hidden, inter, idx, w, [0], _experts(load, E, hidden, inter, bits), sh, 10.0)
    assert_close(load("layer_yr", np.float32).reshape(1, hidden), yr, what="compat layer routed")
    assert_close(load("layer_y", np.uint16).view(np.float16).reshape(1, hidden).astype(np.float64),
                 yo.view(np.float16).astype(np.float64), what="compat layer y")


def test_compat_host_cost(run):
    """Host time per call from C++ at the decode shapes (no synchronization inside the loop)."""
    _, timing = run
    t = timing["host_us_per_call"]
    print("host us per call:", t)
    assert t["moe_layer_config3"] < 10.0 and t["gemm_config1"] < 10.0
