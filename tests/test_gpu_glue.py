"""Router top-k, permutation, ordered reduction, Hadamard and swiglu through the C ABI vs the oracle."""
import itertools

import numpy as np
import pytest

from helpers import assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def hx():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import exl3
    return exl3


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("bsz,E,K", [(1, 288, 8), (4096, 288, 8), (7, 64, 6), (3, 512, 16)])
def test_routing_bit_exact_indices(hx, bsz, E, K):
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(bsz + E)
    s = r.standard_normal((bsz, E)).astype(np.float16)
    s[0, 1] = s[0, 2] = s[0, 3] = np.float16(5.0)  # ties -> lower index first
    if bsz > 1:
        s[1, :] = np.float16(0.0)
        s[1, 5] = np.float16(-0.0)
    idx = torch.empty((bsz, K), dtype=torch.int64, device="cuda")
    w = torch.empty((bsz, K), dtype=torch.float16, device="cuda")
    hx.routing_ds3_nogroup(_dev(s), None, idx, w, bsz, E, K, 2.5)
    torch.cuda.synchronize()
    ri, rw = O.routing(s, K, 2.5)
    assert np.array_equal(idx.cpu().numpy(), ri)
    gw = w.cpu().float().numpy().astype(np.float64)
    rw = rw.view(np.float16).astype(np.float64)
    assert np.abs(gw - rw).max() <= 2 ** -9 * 2.5   # sigmoid via exp: within one fp16 ulp


@pytest.mark.parametrize("bsz,E,K", [(1, 288, 8), (300, 288, 8), (5, 512, 16)])
def test_routing_bias_indices(hx, bsz, E, K):
    """Correction-bias routing (routing.cu:240-326): key sigmoid(logit) + bias, weight the unbiased
    sigmoid; indices equal to the oracle's, weights within one fp16 ulp."""
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(7 * bsz + E)
    s = r.standard_normal((bsz, E)).astype(np.float16)
    b = (r.standard_normal(E) * 0.05).astype(np.float16)
    b[3] = np.float16(4.0)
    idx = torch.empty((bsz, K), dtype=torch.int64, device="cuda")
    w = torch.empty((bsz, K), dtype=torch.float16, device="cuda")
    hx.routing_ds3_nogroup(_dev(s), _dev(b), idx, w, bsz, E, K, 2.5)
    torch.cuda.synchronize()
    ri, rw = O.routing(s, K, 2.5, b)
    assert np.array_equal(idx.cpu().numpy(), ri)
    assert (ri[:, 0] == 3).all()
    gw = w.cpu().float().numpy().astype(np.float64)
    assert np.abs(gw - rw.view(np.float16).astype(np.float64)).max() <= 2 ** -9 * 2.5


@pytest.mark.parametrize("use_topk,act", [(1, 1), (0, 0), (0, 1)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_routing_variants(hx, use_topk, act, with_bias):
    """The sqrt(softplus) activation (ROUTING_ACT_SQRTSP) and the sorting variant (use_topk = 0,
    routing.cu:333-443): indices equal to the oracle's, weights within one fp16 ulp; logits past
    softplus's threshold included."""
    import torch
    from oracle import oracle as O
    bsz, E, K = 64, 288, 8
    r = np.random.default_rng(31 + 2 * act + use_topk)
    s = r.standard_normal((bsz, E)).astype(np.float16)
    s[1, 5] = np.float16(25.0)
    b = (r.standard_normal(E) * 0.05).astype(np.float16) if with_bias else None
    idx = torch.empty((bsz, K), dtype=torch.int64, device="cuda")
    w = torch.empty((bsz, K), dtype=torch.float16, device="cuda")
    hx.routing_ds3_nogroup(_dev(s), _dev(b) if with_bias else None, idx, w, bsz, E, K, 2.5,
                           use_topk=bool(use_topk), act_fn=act)
    torch.cuda.synchronize()
    ri, rw = O.routing(s, K, 2.5, b, use_topk=bool(use_topk), act_fn=act)
    assert np.array_equal(idx.cpu().numpy(), ri)
    gw = w.cpu().float().numpy().astype(np.float64)
    assert np.abs(gw - rw.view(np.float16).astype(np.float64)).max() <= 2 ** -9 * 2.5


@pytest.mark.parametrize("M,E", [(1, 288), (4096, 288), (37, 17)])
def test_permute_bit_exact(hx, M, E):
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(M)
    topk = 8 if E >= 8 else E
    ids = np.stack([r.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    wt = r.random((M, topk)).astype(np.float16)
    cnt = torch.empty(E + 1, dtype=torch.int64, device="cuda")
    ts = torch.empty(M * topk, dtype=torch.int64, device="cuda")
    ws = torch.empty(M * topk, dtype=torch.float16, device="cuda")
    r2s = torch.empty(M * topk, dtype=torch.int64, device="cuda")
    hx.moe_permute(_dev(ids), _dev(wt), M, topk, E, cnt, ts, ws, None, route_to_sorted=r2s)
    torch.cuda.synchronize()
    c0, t0, w0, r0 = O.permute(ids, wt, E)
    assert np.array_equal(cnt.cpu().numpy(), c0)
    assert np.array_equal(ts.cpu().numpy(), t0)
    assert np.array_equal(ws.cpu().numpy().view(np.uint16), w0)
    assert np.array_equal(r2s.cpu().numpy(), r0)


def test_reduce_sorted_reference_fixture(hx):
    """test_deterministic_reductions.cu:49-66: {1e20, -1e20, 1, 1} -> 2.0 for every storage order."""
    import torch
    terms = np.array([1e20, -1e20, 1.0, 1.0], np.float32)
    for perm in itertools.permutations(range(4)):
        contrib = np.zeros((4, 128), np.float32)
        for j in range(4):
            contrib[perm[j]] = terms[j]
        y = torch.empty((1, 128), dtype=torch.float32, device="cuda")
        hx.moe_reduce_sorted(y, _dev(contrib), _dev(np.array(perm, np.int64)), 1, 4, 128)
        torch.cuda.synchronize()
        assert np.all(y.cpu().numpy() == 2.0)


def test_reduce_sorted_random(hx):
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(2)
    M, topk, hidden = 33, 8, 4096
    contrib = r.standard_normal((M * topk, hidden)).astype(np.float32)
    r2s = r.permutation(M * topk).astype(np.int64)
    y = torch.empty((M, hidden), dtype=torch.float32, device="cuda")
    hx.moe_reduce_sorted(y, _dev(contrib), _dev(r2s), M, topk, hidden)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), O.reduce_sorted(contrib, r2s, M, topk))


@pytest.mark.parametrize("mode", ["none", "pre", "post"])
@pytest.mark.parametrize("scale", [1.0, 2.5])
def test_had_r_128(hx, mode, scale):
    """fp16 data: within one fp16 ulp of the exact transform with the reference's rounding points;
    `scale` is multiplied by 1/sqrt(128) inside (hadamard.cu:104)."""
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(3)
    x = (r.integers(-1000, 1001, (64, 256)) / 250.0).astype(np.float16)
    sc = (r.choice([-1.0, 1.0], 256) * r.uniform(0.5, 1.5, 256)).astype(np.float16)
    pre, post = (sc if mode == "pre" else None), (sc if mode == "post" else None)
    out = torch.empty((64, 256), dtype=torch.float16, device="cuda")
    hx.had_r_128(_dev(x), out, None if pre is None else _dev(pre), None if post is None else _dev(post), 64, 256,
                 scale)
    torch.cuda.synchronize()
    ref = O.had_r_128_f16(x, pre, post, scale * 0.088388347648).view(np.float16).astype(np.float64)
    got = out.cpu().float().numpy().astype(np.float64)
    # fp32 butterfly order vs exact: at most one fp16 ulp apart
    assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64) * 1.01)


def _had_exact(x, pre=None, post=None, scale=1.0):
    from scipy.linalg import hadamard
    H = hadamard(128).astype(np.float64)
    v = x.astype(np.float64).reshape(x.shape[0], -1, 128)
    if pre is not None:
        v = v * pre.astype(np.float64).reshape(-1, 128)
    v = (v @ H) * (scale / np.sqrt(128.0))
    if post is not None:
        v = v * post.astype(np.float64).reshape(-1, 128)
    return v.reshape(x.shape)


@pytest.mark.parametrize("mode", ["none", "pre", "post"])
def test_had_r_128_fp32_and_dual(hx, mode):
    """DType::Float data (had_ff_r_128, hadamard.cu:140-166) against scipy's Sylvester matrix in fp64,
    in place, and the dual form on two tensors equal to two single calls."""
    import torch
    r = np.random.default_rng(5)
    x1 = r.standard_normal((33, 384)).astype(np.float32)
    x2 = r.standard_normal((33, 384)).astype(np.float32)
    s1 = r.uniform(0.5, 1.5, 384).astype(np.float16)
    s2 = r.uniform(-1.5, -0.5, 384).astype(np.float16)
    pick = lambda s: (s if mode == "pre" else None, s if mode == "post" else None)
    d = lambda a: None if a is None else _dev(a)
    a = _dev(x1).clone()
    hx.had_r_128(a, a, d(pick(s1)[0]), d(pick(s1)[1]), 33, 384, 0.75)  # in place
    torch.cuda.synchronize()
    ref = _had_exact(x1, *pick(s1), scale=0.75)
    assert np.abs(a.cpu().numpy() - ref).max() <= 1e-5 * np.abs(ref).max()
    o1, o2 = torch.empty_like(a), torch.empty_like(a)
    hx.had_r_128_dual(_dev(x1), o1, d(pick(s1)[0]), d(pick(s1)[1]), _dev(x2), o2, d(pick(s2)[0]), d(pick(s2)[1]),
                      33, 384, 0.75)
    torch.cuda.synchronize()
    assert torch.equal(o1, a)
    ref2 = _had_exact(x2, *pick(s2), scale=0.75)
    assert np.abs(o2.cpu().numpy() - ref2).max() <= 1e-5 * np.abs(ref2).max()
    # fp16 dual equals two single calls bit for bit
    h1, h2 = _dev(x1.astype(np.float16)), _dev(x2.astype(np.float16))
    e1, e2, f1, f2 = (torch.empty_like(h1) for _ in range(4))
    hx.had_r_128(h1, e1, d(pick(s1)[0]), d(pick(s1)[1]), 33, 384)
    hx.had_r_128(h2, e2, d(pick(s2)[0]), d(pick(s2)[1]), 33, 384)
    hx.had_r_128_dual(h1, f1, d(pick(s1)[0]), d(pick(s1)[1]), h2, f2, d(pick(s2)[0]), d(pick(s2)[1]), 33, 384)
    torch.cuda.synchronize()
    assert torch.equal(e1, f1) and torch.equal(e2, f2)


def test_swiglu_clamp(hx):
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(4)
    g = (r.standard_normal(10000) * 6).astype(np.float32)
    u = (r.standard_normal(10000) * 6).astype(np.float32)
    out = torch.empty(10000, dtype=torch.float16, device="cuda")
    hx.swiglu_clamp(_dev(g), _dev(u), out, 10000, 10.0)
    torch.cuda.synchronize()
    ref = O.swiglu_clamp(g, u, 10.0).view(np.float16).astype(np.float64)
    assert_close(out.cpu().float().numpy(), ref, what="swiglu")


def test_moe_max_concurrency_positive():
    """helios::exl3::moe_max_concurrency (exl3_moe.cu:52-56): CU count / 8 of the device."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd._lib import lib
    n = lib.hx_moe_max_concurrency(0)
    assert n == max(1, torch.cuda.get_device_properties(0).multi_processor_count // 8)


@pytest.mark.parametrize("h", [4096, 100])
def test_gather_and_scatter_add_rows(hx, h):
    """The dense-MoE fallback's row glue (glue.cu:48-82): gather is a copy; scatter-add rounds the
    product and the sum once each in fp32, so it equals numpy's float32 arithmetic bit for bit."""
    import torch
    r = np.random.default_rng(h)
    rows, n = 64, 40
    src = r.standard_normal((rows, h)).astype(np.float16)
    idx = r.permutation(rows)[:n].astype(np.int64)
    dst = torch.empty((n, h), dtype=torch.float16, device="cuda")
    hx.gather_rows(_dev(src), _dev(idx), dst, n, h)
    y0 = r.standard_normal((rows, h)).astype(np.float32)
    add = r.standard_normal((n, h)).astype(np.float32)
    w = r.random(n).astype(np.float16)
    y = _dev(y0)
    hx.scatter_add_rows(y, _dev(add), _dev(idx), _dev(w), n, h)
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), src[idx])
    want = y0.copy()
    want[idx] = want[idx] + (w.astype(np.float32)[:, None] * add)
    assert np.array_equal(y.cpu().numpy(), want)


@pytest.mark.parametrize("cols,offset", [(0, 0), (1, 0), (37, 0), (5000, 0), (999, 3)])
def test_pack_signs(hx, cols, offset):
    """hx_pack_signs bit-exact against the oracle; offset > 0 starts the fp16 buffer 2*offset bytes
    into an allocation (not 16-byte aligned: the element-wise load path)."""
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(cols + offset)
    u = r.integers(0, 65536, size=16 * cols + offset, dtype=np.uint16)
    dev = _dev(u.view(np.float16))
    src = dev[offset:]
    packed = torch.full((max(cols, 1),), 0x1234, dtype=torch.int16, device="cuda")
    hx.pack_signs(packed, src, cols)
    torch.cuda.synchronize()
    got = packed.cpu().numpy().view(np.uint16)[:cols]
    assert np.array_equal(got, O.pack_signs(u[offset:], cols))
    if cols == 0:
        assert packed.cpu().numpy().view(np.uint16)[0] == 0x1234  # nothing written


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("n,offset", [(4096, 0), (1, 0), (3_000_001, 0), (100_003, 1)])
def test_count_inf_nan(hx, dtype, n, offset):
    """hx_count_inf_nan against the oracle on values with sprinkled infinities and NaNs (including
    the reference test's +inf / -inf / NaN pattern), aligned and unaligned buffers, and the
    accumulate-into-counts contract (a second call adds the same counts again)."""
    import torch
    from oracle import oracle as O
    r = np.random.default_rng(n + offset)
    if dtype == "f16":
        x = r.standard_normal(n + offset).astype(np.float16)
        specials = np.array([np.inf, -np.inf, np.nan], np.float16)
    else:
        x = r.standard_normal(n + offset).astype(np.float32)
        specials = np.array([np.inf, -np.inf, np.nan], np.float32)
    pos = r.integers(offset, n + offset, size=min(n, 97))
    x[pos] = specials[r.integers(0, 3, size=pos.size)]
    if n >= 4096:
        x[offset + 17], x[offset + 900], x[offset + 2000] = specials[0], specials[1], specials[2]
    want = O.count_inf_nan(x[offset:])
    src = _dev(x)[offset:]
    counts = torch.zeros(2, dtype=torch.int64, device="cuda")
    hx.count_inf_nan(src, counts)
    torch.cuda.synchronize()
    assert tuple(int(v) for v in counts.cpu()) == want
    hx.count_inf_nan(src, counts)
    torch.cuda.synchronize()
    assert tuple(int(v) for v in counts.cpu()) == (2 * want[0], 2 * want[1])
