"""MoE layer parity (router -> permute -> experts -> SiLU-gate -> down -> ordered reduce -> shared
combine) through the C ABI against the CPU oracle."""
import numpy as np
import pytest

from helpers import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import exl3, moe
    return exl3, moe


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


def _run_layer(hx, E, hidden, inter, topk, T, bits, shared_bits, seed, rows=None, bias=False):
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=seed)
    sh = moe.synthetic_dense_mlp(hidden, inter, shared_bits, seed=seed + 1) if shared_bits else None
    layer = moe.MoeLayer(ex, sh, topk=topk)
    r = np.random.default_rng(seed + 2)
    x = r.standard_normal((T, hidden)).astype(np.float16)
    scores = r.standard_normal((T, E)).astype(np.float32).astype(np.float16)
    b = (r.standard_normal(E) * 0.05).astype(np.float16) if bias else None
    y_routed = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    y = layer(torch.from_numpy(x).cuda(), torch.from_numpy(scores).cuda(), y_routed=y_routed,
              bias=torch.from_numpy(b).cuda() if bias else None)
    torch.cuda.synchronize()
    idx, w = O.routing(scores, topk, 2.5, b)
    rows = np.arange(T) if rows is None else np.asarray(rows)
    used = set(int(e) for e in idx[rows].reshape(-1))
    yr_ref, yo_ref = O.moe_rows(x, hidden, inter, idx, w, rows, _oracle_experts(ex, used),
                                _oracle_shared(sh) if sh else None, 10.0)
    got_r = y_routed.cpu().numpy()[rows]
    assert_close(got_r, yr_ref, what=f"routed E={E} T={T}")
    if sh:
        assert_close(y.float().cpu().numpy()[rows], yo_ref.view(np.float16).astype(np.float64), what=f"y E={E} T={T}")
    return ex, y


@pytest.mark.parametrize("T", [1, 3, 8])
def test_moe_decode_small(hx, T):
    _run_layer(hx, E=16, hidden=512, inter=256, topk=4, T=T, bits=2, shared_bits=2, seed=10 + T)


@pytest.mark.parametrize("T", [1, 24])
def test_moe_layer_mcg(hx, T):
    """MCG-codebook experts through MoeLayer(mcg=True), gate/up/down at 2/3/4 bits: the one-token
    decode kernel (T = 1) and the grouped prefill path (T = 24, 96 routed rows), against the oracle's
    layer with codebook 1."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    E, hidden, inter, topk = 16, 512, 256, 4
    ex = moe.ExpertSet.synthetic(E, hidden, inter, (2, 3, 4), seed=900 + T, mul1=False)
    with pytest.raises(ValueError):
        moe.MoeLayer(moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=1), None, topk=topk, mcg=True)
    layer = moe.MoeLayer(ex, None, topk=topk, mcg=True)
    r = np.random.default_rng(901 + T)
    x = r.standard_normal((T, hidden)).astype(np.float16)
    scores = r.standard_normal((T, E)).astype(np.float16)
    y_routed = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    layer(torch.from_numpy(x).cuda(), torch.from_numpy(scores).cuda(), y_routed=y_routed)
    torch.cuda.synchronize()
    idx, w = O.routing(scores, topk, 2.5)
    used = set(int(e) for e in idx.reshape(-1))
    yr_ref, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), _oracle_experts(ex, used), None, 10.0, cb=1)
    assert_close(y_routed.cpu().numpy(), yr_ref, what=f"mcg layer T={T}")


@pytest.mark.parametrize("E,T", [(320, 1), (384, 1), (384, 4), (512, 2)])
def test_moe_decode_many_experts(hx, E, T):
    """Expert counts at and above 320: up to 320 the decode kernel takes every expert's table
    entries with the scores; above it loads the slot's entries after the ranking (both paths)."""
    _run_layer(hx, E=E, hidden=256, inter=256, topk=8, T=T, bits=2, shared_bits=2, seed=600 + E + T)


@pytest.mark.parametrize("E,T", [(288, 1), (288, 4), (384, 1), (64, 12)])
def test_moe_layer_router_bias(hx, E, T):
    """Router correction bias through the layer: the decode kernel's 64-bit-key top-k (with and
    without the slot-table prefetch), and the prefill router for T > 8."""
    _run_layer(hx, E=E, hidden=256, inter=256, topk=8, T=T, bits=2, shared_bits=2, seed=700 + E + T, bias=True)


@pytest.mark.parametrize("E,T,topk", [(288, 1, 8), (288, 4, 8), (288, 8, 8), (64, 2, 8), (512, 1, 8), (64, 1, 32),
                                      (40, 1, 40)])
@pytest.mark.parametrize("bias", [False, True])
def test_decode_router_outputs_bit_exact(hx, E, T, topk, bias):
    """The few-token layer kernel's own top-k: its router outputs (kept in the workspace after the
    64 KiB counter area: indices [T*topk] int64, then the fp16 weights at the next 256-byte
    boundary) equal the stand-alone routing kernel's bit for bit and the oracle's indices
    (routing.cu:211-329), with ties at the top (equal logits: the lower expert first) and, for
    T > 1, a token whose logits are all equal.  E = 512 is past the table prefetch's 320 experts;
    top-40 of 40 selects every expert."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    hidden = 256
    ex = moe.ExpertSet.synthetic(E, hidden, 256, 2, seed=900 + E)
    sh = moe.synthetic_dense_mlp(hidden, 256, 2, seed=901)
    layer = moe.MoeLayer(ex, sh, topk=topk)
    r = np.random.default_rng(902 + E + T + int(bias))
    s = r.standard_normal((T, E)).astype(np.float16)
    s[0, min(10, E - 1)] = s[0, 3] = np.float16(3.0)
    if T > 1:
        s[1, :] = np.float16(0.25)
    b = (r.standard_normal(E) * 0.05).astype(np.float16) if bias else None
    s_d = torch.from_numpy(s).cuda()
    b_d = torch.from_numpy(b).cuda() if bias else None
    x = torch.from_numpy((r.standard_normal((T, hidden)) * 0.5).astype(np.float16)).cuda()
    ws = torch.zeros(layer.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    layer(x, s_d, bias=b_d, ws=ws)
    idx = torch.empty((T, topk), dtype=torch.int64, device="cuda")
    w = torch.empty((T, topk), dtype=torch.float16, device="cuda")
    exl3.routing_ds3_nogroup(s_d, b_d, idx, w, T, E, topk, 2.5)
    torch.cuda.synchronize()
    R = T * topk
    o_idx = 64 * 1024
    o_w = (o_idx + 8 * R + 255) // 256 * 256
    wsh = ws.cpu().numpy()
    got_i = wsh[o_idx:o_idx + 8 * R].view(np.int64).reshape(T, topk)
    got_w = wsh[o_w:o_w + 2 * R].view(np.uint16).reshape(T, topk)
    assert np.array_equal(got_i, idx.cpu().numpy())
    assert np.array_equal(got_w, w.cpu().numpy().view(np.uint16))
    ri, _ = O.routing(s, topk, 2.5, b)
    assert np.array_equal(got_i, ri)
    if not bias and topk < E:
        assert got_i[0, 0] == 3 and got_i[0, 1] == 10
        if T > 1:
            assert list(got_i[1]) == list(range(topk))


def test_empty_batches_are_noops(hx):
    """tokens == 0 / M == 0 through the layer, the grouped call's Python mirror and the linear: no
    launch, no error, even with the null data pointers of empty tensors."""
    import torch
    exl3, moe = hx
    ex = moe.ExpertSet.synthetic(8, 256, 256, 2, seed=1)
    sh = moe.synthetic_dense_mlp(256, 256, 2, seed=2)
    layer = moe.MoeLayer(ex, sh, topk=2)
    x = torch.empty((0, 256), dtype=torch.float16, device="cuda")
    y = layer(x, torch.empty((0, 8), dtype=torch.float16, device="cuda"))
    assert y.shape == (0, 256)
    path = exl3.gemm(torch.empty((0, 256), dtype=torch.float16, device="cuda"), x, sh[0], 0, 256, 256, 2)
    assert path == exl3.HX_GEMM_PATH_GEMV
    torch.cuda.synchronize()


def test_moe_decode_mixed_bits(hx):
    bits = [(2, 3, 4) if e % 2 else (3, 2, 2) for e in range(12)]
    _run_layer(hx, E=12, hidden=256, inter=384, topk=3, T=2, bits=bits, shared_bits=(4, 4, 3), seed=3)


def test_moe_decode_bad_bit_table_is_reported(hx):
    """A per-expert bit table holding a width outside 1..8 (device data the host does not read) is
    reported by the status check as HX_ERR_UNSUPPORTED; the units of that width still take part in
    their handoffs, so the next call with a corrected table runs normally and equals the first."""
    import torch
    from helios_glm53flash_amd._lib import HxError
    exl3, moe = hx
    bits = [(2, 3, 4) if e % 2 else (3, 2, 2) for e in range(12)]
    ex = moe.ExpertSet.synthetic(12, 256, 384, bits, seed=9)
    layer = moe.MoeLayer(ex, moe.synthetic_dense_mlp(256, 384, 2, seed=10), topk=3)
    r = np.random.default_rng(11)
    x = torch.from_numpy(r.standard_normal((2, 256)).astype(np.float16)).cuda()
    s = torch.from_numpy(r.standard_normal((2, 12)).astype(np.float16)).cuda()
    ws = torch.zeros(layer.workspace_bytes(2), dtype=torch.uint8, device="cuda")
    y0 = layer(x, s, ws=ws).clone()
    moe.check_status(ws)
    for which in (9, 11):  # the gate, then the down bit table (tables() keeps 9 pointer arrays first)
        tab = ex._keep[which]
        good = tab.clone()
        tab.fill_(12)
        with pytest.raises(HxError, match="width outside"):  # raised by the call (HX_MOE_SYNC_CHECK) or the check
            layer(x, s, ws=ws)
            moe.check_status(ws)
        tab.copy_(good)
        y1 = layer(x, s, ws=ws)
        moe.check_status(ws)
        assert torch.equal(y0, y1), which


@pytest.mark.parametrize("T", [9, 40])
def test_moe_prefill_small(hx, T):
    _run_layer(hx, E=16, hidden=512, inter=256, topk=4, T=T, bits=2, shared_bits=3, seed=20 + T)


def test_moe_prefill_mixed_bits_no_shared(hx):
    bits = [2 if e < 8 else 3 for e in range(16)]
    _run_layer(hx, E=16, hidden=256, inter=256, topk=8, T=33, bits=bits, shared_bits=None, seed=5)


def test_moe_decode_config3(hx):
    """288 experts + shared, 4096 -> 2048 -> 4096, 2 bits, top-8, 1 token."""
    _run_layer(hx, E=288, hidden=4096, inter=2048, topk=8, T=1, bits=2, shared_bits=2, seed=300)


def test_moe_prefill_config4_sampled(hx):
    """BASELINE config 4 shape at 512 tokens (2/3-bit experts), 6 sampled rows against the oracle."""
    bits = [2 if e < 144 else 3 for e in range(288)]
    _run_layer(hx, E=288, hidden=4096, inter=2048, topk=8, T=512, bits=bits, shared_bits=None, seed=400,
               rows=[0, 1, 77, 200, 311, 511])


def test_moe_grouped_reference_api(hx):
    """moe_grouped with sorted_contributions, then moe_reduce_sorted, equals y += routed sum."""
    import torch
    exl3, moe = hx
    E, hidden, inter, topk = 16, 256, 256, 4
    for T in (2, 24):
        ex = moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=T)
        r = np.random.default_rng(T)
        x = torch.from_numpy(r.standard_normal((T, hidden)).astype(np.float16)).cuda()
        s = torch.from_numpy(r.standard_normal((T, E)).astype(np.float16)).cuda()
        idx = torch.empty((T, topk), dtype=torch.int64, device="cuda")
        w = torch.empty((T, topk), dtype=torch.float16, device="cuda")
        exl3.routing_ds3_nogroup(s, None, idx, w, T, E, topk, 2.5)
        cnt = torch.empty(E + 1, dtype=torch.int64, device="cuda")
        ts = torch.empty(T * topk, dtype=torch.int64, device="cuda")
        wsr = torch.empty(T * topk, dtype=torch.float16, device="cuda")
        r2s = torch.empty(T * topk, dtype=torch.int64, device="cuda")
        exl3.moe_permute(idx, w, T, topk, E, cnt, ts, wsr, None, route_to_sorted=r2s)
        contrib = torch.empty((T * topk, hidden), dtype=torch.float32, device="cuda")
        moe.moe_grouped(x, None, cnt, ts, wsr, ex, T, topk, sorted_contributions=contrib)
        y1 = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
        exl3.moe_reduce_sorted(y1, contrib, r2s, T, topk, hidden)
        y2 = torch.ones((T, hidden), dtype=torch.float32, device="cuda")
        moe.moe_grouped(x, y2, cnt, ts, wsr, ex, T, topk, route_to_sorted=r2s)
        torch.cuda.synchronize()
        # y2 = 1 + sum (accumulate contract): compare up to the fp32 rounding of that addition
        assert float((y2 - (1.0 + y1)).abs().max()) <= float(y1.abs().max()) * 2 ** -22


@pytest.mark.parametrize("T", [4, 8])
def test_moe_decode_config3_several_tokens(hx, T):
    """Config-3 shape with 4 and 8 tokens (up to 64 routed slots + shared: more units than one round of
    resident workgroups), 2 sampled tokens against the oracle."""
    _run_layer(hx, E=288, hidden=4096, inter=2048, topk=8, T=T, bits=2, shared_bits=2, seed=500 + T,
               rows=[0, T - 1])


@pytest.mark.parametrize("act", [1, 2])
@pytest.mark.parametrize("T", [1, 5, 24, 40])
def test_moe_grouped_activations(hx, act, T):
    """act_function 1 (tanh-form GELU) and 2 (non-gated relu2) through hx_moe_grouped, on the
    few-token decode kernel (T <= 8) and the grouped MFMA path.  For relu2 the gate weights and
    scales are filled with +inf first: any read of them would poison the output."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    E, hidden, inter, topk = 16, 512, 256, 4
    ex = moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=900 + T + act)
    r = np.random.default_rng(900 + T)
    xh = (r.standard_normal((T, hidden)) * 0.5).astype(np.float16)
    sh = r.standard_normal((T, E)).astype(np.float16)
    idx, w = O.routing(sh, topk, 2.5)
    used = set(int(e) for e in idx.reshape(-1))
    oe = _oracle_experts(ex, used)
    if act == 2:
        for e in range(E):
            ex.suh[0][e].fill_(float("inf"))
            ex.svh[0][e].fill_(float("inf"))
            ex.trellis[0][e].fill_(-1)
    x = torch.from_numpy(xh).cuda()
    idx_d = torch.from_numpy(idx).cuda()
    w_d = torch.from_numpy(w.view(np.float16)).cuda()
    cnt = torch.empty(E + 1, dtype=torch.int64, device="cuda")
    ts = torch.empty(T * topk, dtype=torch.int64, device="cuda")
    wsr = torch.empty(T * topk, dtype=torch.float16, device="cuda")
    r2s = torch.empty(T * topk, dtype=torch.int64, device="cuda")
    exl3.moe_permute(idx_d, w_d, T, topk, E, cnt, ts, wsr, None, route_to_sorted=r2s)
    y = torch.zeros((T, hidden), dtype=torch.float32, device="cuda")
    moe.moe_grouped(x, y, cnt, ts, wsr, ex, T, topk, act_limit=10.0, route_to_sorted=r2s, act_function=act)
    torch.cuda.synchronize()
    ref, _ = O.moe_rows(xh.view(np.uint16), hidden, inter, idx, w, np.arange(T), oe, None, 10.0, act=act)
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    assert_close(got, ref, what=f"act={act} T={T}")


@pytest.mark.parametrize("topk", [1, 2, 6, 16])
def test_moe_prefill_topk_variants(hx, topk):
    """The matrix-core combine serves topk dividing 16 (1, 2, 16 here, besides 4 and 8 above), the
    per-token combine any other topk (6)."""
    _run_layer(hx, E=32, hidden=256, inter=256, topk=topk, T=20, bits=2, shared_bits=2, seed=950 + topk)


@pytest.mark.parametrize("cb", [2, 1])
@pytest.mark.parametrize("T", [5, 160, 404])
def test_moe_grouped_every_bit_width(hx, cb, T):
    """hx_moe_grouped with per-expert bit widths that cover 1..8 in every projection (expert e:
    gate 1 + e % 8, up 1 + (e + 3) % 8, down 1 + (e + 5) % 8), codebook mul1 (cb 2) and MCG (cb 1),
    on the few-token decode kernel (T = 5) and the grouped MFMA path (T = 160, 404).  Tokens 0..3
    route to every expert.  At T = 160 the other tokens favour experts 0..3, which then take 128-row
    tiles besides the 32-row ones of the others; at T = 404 token t >= 4 routes to experts
    (t + k) % 8, k < 4, so experts 0..7 (every width in every projection) get 201 or 200 rows: a
    128-row tile and a 96-row tile each."""
    import torch
    from oracle import oracle as O
    exl3, moe = hx
    E, hidden, inter, topk = 16, 512, 256, 4
    bits = [(1 + e % 8, 1 + (e + 3) % 8, 1 + (e + 5) % 8) for e in range(E)]
    ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=1000 + T + cb, mul1=(cb == 2))
    r = np.random.default_rng(1000 + T)
    xh = (r.standard_normal((T, hidden)) * 0.5).astype(np.float16)
    s = r.standard_normal((T, E))
    for t in range(4):  # tokens 0..3 route to experts 4t..4t+3: every expert, so every width, is used
        s[t, 4 * t:4 * t + 4] += 6.0
    if T == 404:
        for t in range(4, T):
            s[t, [(t + k) % 8 for k in range(4)]] += 6.0
    else:
        s[4:, :4] += 3.0  # the hot experts of the longer batch
    sh = s.astype(np.float16)
    idx, w = O.routing(sh, topk, 2.5)
    used = set(int(e) for e in idx.reshape(-1))
    assert len(used) == E, "every expert (so every width) is routed"
    if T == 404:
        c = np.bincount(idx.reshape(-1), minlength=E)
        for p in range(3):
            assert {bits[e][p] for e in range(E) if 64 < c[e] % 128 <= 96} == set(range(1, 9)), c
    x = torch.from_numpy(xh).cuda()
    idx_d = torch.from_numpy(idx).cuda()
    w_d = torch.from_numpy(w.view(np.float16)).cuda()
    cnt = torch.empty(E + 1, dtype=torch.int64, device="cuda")
    ts = torch.empty(T * topk, dtype=torch.int64, device="cuda")
    wsr = torch.empty(T * topk, dtype=torch.float16, device="cuda")
    r2s = torch.empty(T * topk, dtype=torch.int64, device="cuda")
    exl3.moe_permute(idx_d, w_d, T, topk, E, cnt, ts, wsr, None, route_to_sorted=r2s)
    y = torch.zeros((T, hidden), dtype=torch.float32, device="cuda")
    moe.moe_grouped(x, y, cnt, ts, wsr, ex, T, topk, act_limit=10.0, route_to_sorted=r2s, mcg=(cb == 1))
    torch.cuda.synchronize()
    ref, _ = O.moe_rows(xh.view(np.uint16), hidden, inter, idx, w, np.arange(T), _oracle_experts(ex, used), None,
                        10.0, cb=cb)
    got = y.cpu().numpy()
    assert np.isfinite(got).all()
    assert_close(got, ref, what=f"every width, cb={cb}, T={T}")
