"""Router front end: hx_gemm_nt_f16 (glue2.cu:9-65,165-182) against an fp64 matmul, and a MoE layer fed
by its own router weight against the same layer fed precomputed logits."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_mod():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _ulps(a16, b16):
    """|a - b| in units of the fp16 spacing (same-sign finite values)."""
    ai = a16.view(np.int16).astype(np.int32)
    bi = b16.view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


@pytest.mark.parametrize("M,N,K", [(1, 288, 4096), (5, 288, 4096), (8, 100, 256), (300, 288, 4096), (37, 70, 96)])
def test_gemm_nt_f16_fp16_out(torch_mod, M, N, K):
    torch = torch_mod
    from helios_glm53flash_amd import exl3
    r = np.random.default_rng(M * 1000 + N)
    x = r.standard_normal((M, K)).astype(np.float16)
    w = (r.standard_normal((N, K)) * 0.02).astype(np.float16)
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    exl3.gemm_nt_f16(y, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), M, N, K)
    torch.cuda.synchronize()
    ref64 = x.astype(np.float64) @ w.astype(np.float64).T
    ref = ref64.astype(np.float16)
    got = y.cpu().numpy()
    # fp32 accumulation in another order than fp64: the error is the fp16 rounding (at most one
    # spacing of the exact value) plus fp32 summation noise, bounded by the sum of |products|
    mag = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    spacing = np.spacing(np.abs(ref64).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref64) <= spacing + 2.0 ** -20 * mag)
    d = _ulps(got, ref)
    assert (d > 0).mean() < 0.01, (d > 0).mean()


@pytest.mark.parametrize("M", [1, 200])
def test_gemm_nt_f16_fp32_out_and_add(torch_mod, M):
    torch = torch_mod
    from helios_glm53flash_amd import exl3
    N, K = 96, 512
    r = np.random.default_rng(M)
    x = r.standard_normal((M, K)).astype(np.float16)
    w = r.standard_normal((N, K)).astype(np.float16)
    ref = x.astype(np.float64) @ w.astype(np.float64).T
    y = torch.ones((M, N), dtype=torch.float32, device="cuda")
    exl3.gemm_nt_f16(y, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), M, N, K, y_fp32=True, add=True)
    torch.cuda.synchronize()
    tol = 1e-5 * np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T + 1e-6
    assert np.all(np.abs(y.cpu().numpy() - (1.0 + ref)) <= tol + 2 ** -22 * np.abs(1.0 + ref))
    exl3.gemm_nt_f16(y, torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), M, N, K, y_fp32=True)
    torch.cuda.synchronize()
    assert np.all(np.abs(y.cpu().numpy() - ref) <= tol)


@pytest.mark.parametrize("T", [1, 20])
def test_layer_with_router_weight(torch_mod, T):
    torch = torch_mod
    from helios_glm53flash_amd import exl3, moe
    E, hidden, inter = 16, 512, 256
    ex = moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=T)
    r = np.random.default_rng(T)
    wr = torch.from_numpy((r.standard_normal((E, hidden)) * 0.05).astype(np.float16)).cuda()
    x = torch.from_numpy(r.standard_normal((T, hidden)).astype(np.float16)).cuda()
    layer = moe.MoeLayer(ex, None, topk=4, router_weight=wr)
    y1 = layer(x)
    scores = torch.empty((T, E), dtype=torch.float16, device="cuda")
    exl3.gemm_nt_f16(scores, x, wr, T, E, hidden)
    y2 = layer(x, scores)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)


@pytest.mark.parametrize("bias,act", [(False, 0), (True, 0), (False, 1)])
def test_routing_ds3_nogroup_hidden(torch_mod, bias, act):
    """Decode fast path (routing.cuh:51-66): the router GEMV (routing_gemv) within one fp16 spacing of
    the fp64 dot products plus fp32 noise, and the top-k indices bit-exact against the oracle's
    routing of the GEMV's own scores (weights within one fp16 ulp), at E = 288, K = 8, k = 4096."""
    torch = torch_mod
    from helios_glm53flash_amd import exl3
    from oracle import oracle as O
    E, k, K = 288, 4096, 8
    r = np.random.default_rng(91 + 7 * act + bias)
    x = r.standard_normal(k).astype(np.float16)
    gate = (r.standard_normal((E, k)) * 0.02).astype(np.float16)
    b = (r.standard_normal(E) * 0.05).astype(np.float16) if bias else None
    scores = torch.empty(E, dtype=torch.float16, device="cuda")
    idx = torch.empty(K, dtype=torch.int64, device="cuda")
    w = torch.empty(K, dtype=torch.float16, device="cuda")
    exl3.routing_ds3_nogroup_hidden(torch.from_numpy(x).cuda(), torch.from_numpy(gate).cuda(), scores,
                                    torch.from_numpy(b).cuda() if bias else None, idx, w, k, E, K, 2.5, act)
    torch.cuda.synchronize()
    ref64 = gate.astype(np.float64) @ x.astype(np.float64)
    got = scores.cpu().numpy()
    mag = np.abs(gate.astype(np.float64)) @ np.abs(x.astype(np.float64))
    spacing = np.spacing(np.abs(ref64).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got.astype(np.float64) - ref64) <= spacing + 2.0 ** -20 * mag)
    ridx, rw = O.routing(got[None, :], K, 2.5, b, True, act)
    assert np.array_equal(idx.cpu().numpy(), ridx[0])
    dw = np.abs(w.cpu().numpy().astype(np.float64) - rw[0].view(np.float16).astype(np.float64))
    assert dw.max() <= 2.0 ** -9 * 2.5
    # routing_gemv alone writes the same scores
    s2 = torch.empty(E, dtype=torch.float16, device="cuda")
    exl3.routing_gemv(torch.from_numpy(x).cuda(), torch.from_numpy(gate).cuda(), s2, k, E)
    torch.cuda.synchronize()
    assert torch.equal(s2, scores)
