"""BASELINE configs at their real workloads, through the C ABI, against the CPU oracle:
config 4 (4096-token prefill, Zipf(1.1) routing, 2/3-bit experts), config 5 (5-bit lm_head at
4096 -> 151552, the 42-layer decode sweep), config 2 at every M, and structured inputs on which the
per-weight rounding that the fused codebook-2 paths skip could accumulate."""
import numpy as np
import pytest

from helpers import assert_close, expert_contrib_numpy, make_linear, make_x, zipf_scores

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import exl3, moe
    return exl3, moe


def _dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.cuda()


def _host(t):
    import torch
    return t.cpu().view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.int16 else t.cpu().numpy()


def _oracle_experts(ex, used):
    dummy = np.zeros(16, np.uint16)
    out = {"trellis": [], "suh": [], "svh": [], "bits": []}
    for p in range(3):
        out["trellis"].append([_host(ex.trellis[p][e]) if e in used else dummy for e in range(ex.num_experts)])
        out["suh"].append([_host(ex.suh[p][e]).view(np.uint16) if e in used else dummy for e in range(ex.num_experts)])
        out["svh"].append([_host(ex.svh[p][e]).view(np.uint16) if e in used else dummy for e in range(ex.num_experts)])
        out["bits"].append(np.array(ex.bits[p], np.int32))
    return out


def _oracle_shared(sh):
    return {"trellis": [_host(w.trellis) for w in sh], "suh": [_host(w.suh).view(np.uint16) for w in sh],
            "svh": [_host(w.svh).view(np.uint16) for w in sh], "bits": [w.bits for w in sh]}


def _al(v):
    return (v + 255) & ~255


@pytest.fixture(scope="module")
def config4(hx):
    """Config 4 at its workload, run once: 4096 tokens, top-8 of 288 with Zipf(1.1) popularity,
    experts 0-143 2-bit and 144-287 3-bit.  Returns the layer's inputs, y_routed, its workspace's
    router outputs and permutation, and the per-route contributions of the same routing through
    moe_grouped(sorted_contributions) (the same grouped gate/up and down kernels)."""
    import torch
    exl3, moe = hx
    E, hidden, inter, topk, T = 288, 4096, 2048, 8, 4096
    bits = [2 if e < 144 else 3 for e in range(E)]
    ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=4000)
    layer = moe.MoeLayer(ex, None, topk=topk)
    scores = zipf_scores(T, E, 1.1, seed=11)
    x = make_x(4001, T, hidden)
    ws = torch.zeros(layer.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    y_routed = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    layer(_dev(x), _dev(scores), y_routed=y_routed, ws=ws)
    torch.cuda.synchronize()
    # router outputs and permutation in the workspace (layout of MoeWs::plan: after the 64 KiB
    # counter area, idx int64[R], w fp16[R], expert_count int64[E+1], token_sorted int64[R],
    # weight_sorted fp16[R], route_to_sorted int64[R], each 256-byte aligned)
    R = T * topk
    off_idx = 65536
    off_w = _al(off_idx + 8 * R)
    off_cnt = _al(off_w + 2 * R)
    off_ts = _al(off_cnt + 8 * (E + 1))
    off_ws = _al(off_ts + 8 * R)
    off_r2s = _al(off_ws + 2 * R)
    raw = ws[:off_r2s + 8 * R].cpu().numpy()
    d = dict(E=E, hidden=hidden, inter=inter, topk=topk, T=T, ex=ex, x=x, scores=scores,
             y_routed=y_routed.cpu().numpy(),
             idx=raw[off_idx:off_idx + 8 * R].view(np.int64).reshape(T, topk).copy(),
             w=raw[off_w:off_w + 2 * R].view(np.uint16).reshape(T, topk).copy(),
             cnt=raw[off_cnt:off_cnt + 8 * (E + 1)].view(np.int64).copy(),
             ts=raw[off_ts:off_ts + 8 * R].view(np.int64).copy(),
             wsr=raw[off_ws:off_ws + 2 * R].view(np.uint16).copy(),
             r2s=raw[off_r2s:off_r2s + 8 * R].view(np.int64).copy())
    contrib = torch.empty((R, hidden), dtype=torch.float32, device="cuda")
    moe.moe_grouped(_dev(x), None, _dev(d["cnt"]), _dev(d["ts"]), _dev(d["wsr"], torch.float16), ex, T, topk,
                    sorted_contributions=contrib)
    torch.cuda.synchronize()
    d["contrib"] = contrib.cpu().numpy()
    return d


def test_moe_prefill_config4_zipf(hx, config4):
    """Config 4: the layer's own router indices and chunked permutation (read from its workspace)
    are bit-exact for all 4096 tokens, its weights within one fp16 ulp; sampled rows (the hottest
    expert's first and last token, a token routed only to experts with at most 64 rows, a token of an
    expert with 65-128 rows, and fixed tokens) match the oracle."""
    from oracle import oracle as O
    c4 = config4
    E, hidden, inter, topk, T, x = c4["E"], c4["hidden"], c4["inter"], c4["topk"], c4["T"], c4["x"]
    idx, w = O.routing(c4["scores"], topk, 2.5)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    # the workload has the shapes the prefill tiles are chosen for
    assert counts.max() > 256 and ((counts > 64) & (counts <= 128)).any()
    assert np.array_equal(c4["idx"], idx)
    # weights: sigmoid through exp, within one fp16 ulp of the oracle's (as the router test)
    lw = c4["w"]
    assert np.abs(lw.view(np.float16).astype(np.float64) - w.view(np.float16).astype(np.float64)).max() <= 2 ** -9 * 2.5
    cnt, ts, wsr, r2s = O.permute(idx, lw, E)  # the permutation of the layer's own weights, bit-exact
    assert np.array_equal(c4["cnt"], cnt)
    assert np.array_equal(c4["ts"], ts)
    assert np.array_equal(c4["wsr"], wsr)
    assert np.array_equal(c4["r2s"], r2s)

    hot = int(counts.argmax())
    hot_tokens = np.nonzero((idx == hot).any(axis=1))[0]
    cold = np.nonzero(counts[idx].max(axis=1) <= 64)[0]
    mid_e = int(np.nonzero((counts > 64) & (counts <= 128))[0][0])
    mid_tok = int(np.nonzero((idx == mid_e).any(axis=1))[0][-1])
    rows = sorted({int(hot_tokens[0]), int(hot_tokens[-1]), mid_tok, 0, 2047, T - 1}
                  | ({int(cold[0])} if len(cold) else set()))
    used = set(int(e) for e in idx[rows].reshape(-1))
    ref, _ = O.moe_rows(x, hidden, inter, idx, w, rows, _oracle_experts(c4["ex"], used), None, 10.0)
    assert_close(c4["y_routed"][rows], ref, what=f"config 4 rows {rows}")


def test_moe_prefill_config4_every_job(hx, config4):
    """Config 4, every grouped-GEMM job: the prefill cuts each expert's rows into 128-row jobs (the
    remainder as a 32-, 64-, 96- or 128-row tile); the first and last row of every (expert, job) pair are
    compared against the dense numpy expert (decoded W_hat from the oracle's reconstruct, the fp16
    rounding points of exl3_moe_kernel.cuh:85-262, pinned by test_moe_rows_matches_dense_numpy) as
    per-route contributions, and the layer's y_routed equals the rank-order sum of those
    contributions for all 4096 tokens."""
    import concurrent.futures as cf
    import os
    from oracle import oracle as O
    c4 = config4
    E, hidden, inter, topk, T, ex = c4["E"], c4["hidden"], c4["inter"], c4["topk"], c4["T"], c4["ex"]
    cnt, ts, wsr, r2s, contrib = c4["cnt"], c4["ts"], c4["wsr"], c4["r2s"], c4["contrib"]
    off = np.concatenate([[0], np.cumsum(cnt[:E])])
    jobs = []  # (expert, first sorted row, last sorted row)
    for e in range(E):
        for j0 in range(0, int(cnt[e]), 128):
            jobs.append((e, int(off[e]) + j0, int(off[e]) + min(j0 + 128, int(cnt[e])) - 1))
    # the workload has remainder jobs of every tile height, and 3-bit remainders off the 32-row grid
    rem = [int(cnt[e]) % 128 for e in range(E)]
    assert any(0 < r <= 32 for r in rem) and any(32 < r <= 64 for r in rem)
    assert any(64 < r <= 96 for r in rem) and any(r > 96 for r in rem)
    assert any(e >= 144 and cnt[e] > 128 and cnt[e] % 32 for e in range(E))
    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]

    def check_expert(e):
        pos = sorted({p for (je, a, b) in jobs if je == e for p in (a, b)})
        if not pos:
            return e, [], None, None
        Ws = []
        for p, (K, N) in enumerate(shapes):
            tr = _host(ex.trellis[p][e])
            Ws.append(O.reconstruct(tr, K, N, ex.bits[p][e], 2).view(np.float16).astype(np.float64))
        su = [_host(ex.suh[p][e]).astype(np.float64) for p in range(3)]
        sv = [_host(ex.svh[p][e]).astype(np.float64) for p in range(3)]
        tok = ts[pos]  # token_sorted holds token indices
        wt = wsr[pos].view(np.float16).astype(np.float64)
        ref = expert_contrib_numpy(c4["x"][tok], *Ws, su, sv, wt, 10.0)
        return e, pos, ref, contrib[pos]

    got_all, ref_all, covered = [], [], 0
    with cf.ThreadPoolExecutor(min(16, os.cpu_count() or 1)) as pool:
        for e, pos, ref, got in pool.map(check_expert, range(E)):
            if pos:
                ref_all.append(ref)
                got_all.append(got)
                covered += sum(1 for (je, _, _) in jobs if je == e)
    assert covered == len(jobs) and len(jobs) > 400, (covered, len(jobs))
    assert_close(np.concatenate(got_all), np.concatenate(ref_all), what=f"config 4, {len(jobs)} jobs' end rows")
    # the layer's combine: y_routed[t] = sum over ranks k of contribution row r2s[t * topk + k]
    y_sum = contrib[r2s.reshape(T, topk)].astype(np.float64).sum(axis=1)
    assert_close(c4["y_routed"], y_sum, tol=1e-5, what="config 4 y_routed vs contributions")


@pytest.mark.parametrize("M", [1, 512])
def test_lm_head_5bit_sampled_columns(hx, M):
    """Config 5a: the 5-bit lm_head at its real shape (K=4096 -> N=151552), GEMV (M=1) and MFMA
    (M=512); sampled 128-column groups against the oracle (each group's output transform depends only
    on its own columns, so a tile-column slice of the weight is an exact sub-problem)."""
    import torch
    from oracle import oracle as O
    exl3, _ = hx
    K, N, bits = 4096, 151552, 5
    tr, suh, svh = make_linear(500 + M, K, N, bits)
    x = make_x(501 + M, M, K)
    w = exl3.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), exl3.MUL1)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    a_had = torch.empty((M, K), dtype=torch.float16, device="cuda") if M > exl3.GEMV_MAX_M else None
    path = exl3.gemm(y, _dev(x), w, M, N, K, bits, True, a_had=a_had)
    torch.cuda.synchronize()
    assert path == (exl3.HX_GEMM_PATH_GEMV if M == 1 else exl3.HX_GEMM_PATH_MFMA)
    got = y.cpu().numpy()
    rows = np.arange(M) if M <= 16 else np.array([0, 1, 127, 128, 300, 511])
    for g in (0, 1, 600, N // 128 - 1):
        sl = slice(128 * g, 128 * g + 128)
        sub = np.ascontiguousarray(tr[:, 8 * g:8 * g + 8, :])
        ref = O.linear(x[rows], sub, suh, np.ascontiguousarray(svh[sl]), K, 128, bits, 2, out_f16=False)
        assert_close(got[rows, sl], ref, what=f"lm_head 5-bit M={M} group {g}")


def test_config2_every_m(hx):
    """Config 2: K=4096 -> N=12288, 4-bit, at M = 1, 4 and 8 against the oracle."""
    import torch
    from oracle import oracle as O
    exl3, _ = hx
    K, N, bits = 4096, 12288, 4
    tr, suh, svh = make_linear(240, K, N, bits)
    w = exl3.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), exl3.MUL1)
    for M in (1, 4, 8):
        x = make_x(241 + M, M, K)
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        assert exl3.gemm(y, _dev(x), w, M, N, K, bits, True) == exl3.HX_GEMM_PATH_GEMV
        torch.cuda.synchronize()
        assert_close(y.cpu().numpy(), O.linear(x, tr, suh, svh, K, N, bits, 2), what=f"config 2 M={M}")


def test_decode_sweep_42_layers(hx):
    """Config 5b: 42 decode layers of 288 routed 2-bit experts and one 2-bit shared expert each, all
    resident, run back to back on one stream with independent seeded routing per layer.  Sampled
    layers equal the same layer run alone (bit for bit), and the full fp16 y (routed + shared) of
    three layers matches the oracle."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    E, hidden, inter, topk, L = 288, 4096, 2048, 8, 42
    layers = [moe.MoeLayer(moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=7000 + i),
                           moe.synthetic_dense_mlp(hidden, inter, 2, seed=8000 + i), topk=topk)
              for i in range(L)]
    r = np.random.default_rng(42)
    xs = [r.standard_normal((1, hidden)).astype(np.float16) for _ in range(L)]
    ss = [r.standard_normal((1, E)).astype(np.float16) for _ in range(L)]
    xd = [_dev(v) for v in xs]
    sd = [_dev(v) for v in ss]
    ws = torch.zeros(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    outs = [torch.empty((1, hidden), dtype=torch.float16, device="cuda") for _ in range(L)]
    for i in range(L):
        layers[i](xd[i], sd[i], y=outs[i], ws=ws)
    torch.cuda.synchronize()
    moe.check_status(ws)
    for i in (0, 17, L - 1):
        alone = torch.empty((1, hidden), dtype=torch.float16, device="cuda")
        layers[i](xd[i], sd[i], y=alone, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(alone, outs[i]), f"layer {i} differs from its run in the sweep"
    for i in (5, 30, L - 2):
        idx, w = O.routing(ss[i], topk, 2.5)
        used = set(int(e) for e in idx.reshape(-1))
        _, ref = O.moe_rows(xs[i], hidden, inter, idx, w, [0], _oracle_experts(layers[i].experts, used),
                            _oracle_shared(layers[i].shared), 10.0)
        assert_close(outs[i].float().cpu().numpy(), ref.view(np.float16).astype(np.float64), what=f"sweep layer {i}")


def _structured_inputs(K, suh, seed):
    """Activations on which per-weight rounding errors add up instead of averaging out:
      - ones: x = 1;
      - one-hot x (a single k): the transformed row is one 128-block of +-1/sqrt(128);
      - constant a: x = suh[k] at the first k of every 128-block, so H(x . suh) = 1/sqrt(128)
        everywhere and the output is the plain column sum of the decoded weights;
      - one-hot a: x = suh . H(e_j), so the transformed row is e_j (up to fp16 rounding of x) and
        the output is one decoded weight row."""
    import scipy.linalg
    H = scipy.linalg.hadamard(128) / np.sqrt(128.0)
    rows = []
    rows.append(np.ones(K))
    oh = np.zeros(K)
    oh[(seed * 97) % K] = 1.0
    rows.append(oh)
    ca = np.zeros(K)
    ca[::128] = suh.astype(np.float64)[::128]
    rows.append(ca)
    j = (seed * 31) % K
    b = j // 128
    ha = np.zeros(K)
    ha[128 * b:128 * b + 128] = H[:, j % 128] * suh.astype(np.float64)[128 * b:128 * b + 128]
    rows.append(ha)
    return np.stack(rows).astype(np.float16)


@pytest.mark.parametrize("M_pad", [0, 60])
def test_linear_structured_inputs(hx, M_pad):
    """Config-1 linear (K=4096, N=2048, 2-bit, codebook 2) on the structured inputs, through the
    fused GEMV (4 rows) and, padded with random rows to 64, the MFMA tile path."""
    import torch
    from oracle import oracle as O
    exl3, _ = hx
    K, N, bits = 4096, 2048, 2
    tr, suh, svh = make_linear(1, K, N, bits)
    x = _structured_inputs(K, suh, seed=3)
    if M_pad:
        x = np.concatenate([x, make_x(9, M_pad, K)])
    M = x.shape[0]
    w = exl3.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), exl3.MUL1)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    a_had = torch.empty((M, K), dtype=torch.float16, device="cuda") if M > exl3.GEMV_MAX_M else None
    exl3.gemm(y, _dev(x), w, M, N, K, bits, True, a_had=a_had)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    ref = O.linear(x, tr, suh, svh, K, N, bits, 2)
    for m in range(4):  # each structured row against its own scale
        assert_close(got[m], ref[m], what=f"structured input {m} (M={M})")


def test_moe_decode_structured_inputs(hx):
    """Config-3 layer (288 experts + shared, 2-bit, 1 token) on each structured input."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    E, hidden, inter, topk = 288, 4096, 2048, 8
    ex = moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=310)
    sh = moe.synthetic_dense_mlp(hidden, inter, 2, seed=311)
    layer = moe.MoeLayer(ex, sh, topk=topk)
    r = np.random.default_rng(312)
    scores = r.standard_normal((1, E)).astype(np.float16)
    idx, w = O.routing(scores, topk, 2.5)
    used = set(int(e) for e in idx.reshape(-1))
    oe, osh = _oracle_experts(ex, used), _oracle_shared(sh)
    suh_g = _host(ex.suh[0][int(idx[0, 0])]).view(np.float16)
    for m, xv in enumerate(_structured_inputs(hidden, suh_g, seed=5)):
        x = xv[None, :]
        y_routed = torch.empty((1, hidden), dtype=torch.float32, device="cuda")
        y = layer(_dev(x), _dev(scores), y_routed=y_routed)
        torch.cuda.synchronize()
        yr, yo = O.moe_rows(x, hidden, inter, idx, w, [0], oe, osh, 10.0)
        assert_close(y_routed.cpu().numpy(), yr, what=f"structured {m} routed")
        assert_close(y.float().cpu().numpy(), yo.view(np.float16).astype(np.float64), what=f"structured {m} y")


@pytest.mark.parametrize("K", [640, 1152])
def test_gemv_k_without_512_divisor(hx, K):
    """K with no multiple-of-128 divisor in [512, K) except K itself: the split-K plan keeps its
    chunk floor instead of shrinking past it."""
    import torch
    from oracle import oracle as O
    exl3, _ = hx
    N, bits = 1024, 3
    tr, suh, svh = make_linear(K, K, N, bits)
    x = make_x(K + 1, 2, K)
    w = exl3.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), exl3.MUL1)
    y = torch.empty((2, N), dtype=torch.float32, device="cuda")
    exl3.gemm(y, _dev(x), w, 2, N, K, bits, True)
    torch.cuda.synchronize()
    assert_close(y.cpu().numpy(), O.linear(x, tr, suh, svh, K, N, bits, 2), what=f"K={K}")
