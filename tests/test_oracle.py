"""Pins the CPU oracle (oracle/exl3_oracle.c) independently of its own formulas.

Each check below comes from something other than the oracle's code: numpy/scipy arithmetic,
the reference's own layout model and test fixtures, or invariants of the mathematics.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import scipy.linalg
import scipy.special

from oracle import oracle as O
from helpers import expert_contrib_numpy, make_linear, make_x

GOLD = Path(__file__).resolve().parent / "golden"


# ---------------------------------------------------------------- fp16

def test_fp16_roundtrip_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = h.view(np.float16).astype(np.float64)
    for i in range(0, 65536, 1):
        v = f[i]
        if np.isnan(v):
            continue
        assert O.d2h(float(v)) == h[i]
        assert O.h2d(int(h[i])) == v


def test_fp16_rounding_matches_numpy():
    r = np.random.default_rng(1)
    vals = np.concatenate([r.standard_normal(20000) * 10.0 ** r.integers(-8, 5, 20000),
                           [65504.0, 65519.99, 65520.0, 6.0e-8, 2.98e-8, 2.9802322387695312e-08]])
    for v in vals:
        assert O.d2h(float(v)) == np.array(v, np.float64).astype(np.float16).view(np.uint16), v


# ---------------------------------------------------------------- bitstream

def _stream_bits(tile_u16: np.ndarray) -> np.ndarray:
    """Stream bits straight from the reference packer's definition (pack.cu:27-53): uint16 words
    MSB-first, then each uint32 pair half-swapped.  So the stream is the big-endian bit order of
    the little-endian uint32 words."""
    w32 = tile_u16.view(np.uint32)
    return np.unpackbits(w32.astype(">u4").view(np.uint8))


@pytest.mark.parametrize("bits", range(1, 9))
def test_window_matches_bitstream_definition(bits):
    r = np.random.default_rng(bits)
    tile = r.integers(0, 65536, 16 * bits, dtype=np.uint16)
    sb = _stream_bits(tile)
    total = 256 * bits
    for p in range(256):
        end = (p + 1) * bits
        idx = [(end - 16 + i) % total for i in range(16)]
        want = int("".join(str(b) for b in sb[idx]), 2)
        assert O.window(tile, bits, p) == want


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8])
def test_window_impulse(bits):
    """A single set stream bit b appears in exactly the windows whose 16-bit span covers b, at
    bit position (end - 1 - b) of each (MSB-first)."""
    total = 256 * bits
    for b in [0, 1, 15, 16, 31, 32, total - 1, total // 2 + 3]:
        words = np.zeros(8 * bits, np.uint32)
        words[b // 32] = np.uint32(1) << np.uint32(31 - b % 32)
        tile = words.view(np.uint16)
        for p in range(256):
            end = (p + 1) * bits
            d = (end - 1 - b) % total
            want = (1 << d) if d < 16 else 0
            assert O.window(tile, bits, p) == want, (bits, b, p)


@pytest.mark.parametrize("bits", range(1, 9))
def test_pack_roundtrip_symbols(bits):
    r = np.random.default_rng(100 + bits)
    sym = r.integers(0, 1 << bits, 256)
    tile = O.pack_tile(sym, bits)
    win = O.unpack_tile(tile, bits)
    assert np.array_equal(win & ((1 << bits) - 1), sym)
    # window p = previous symbols concatenated (16 bits of history, tail-biting)
    for p in range(256):
        w = 0
        nsym = (16 + bits - 1) // bits
        for q in range(p - nsym + 1, p + 1):
            w = (w << bits) | int(sym[q % 256])
        assert int(win[p]) == w & 0xFFFF


def test_pack_worked_example():
    """2-bit symbols 3,0,1,2,... -> stream 11 00 01 10 ...; first uint16 of the MSB-first stream
    lands in the high half of the first uint32 (SWAP16)."""
    sym = np.zeros(256, np.int64)
    sym[:8] = [3, 0, 1, 2, 3, 3, 0, 0]
    tile = O.pack_tile(sym, 2)
    w0 = int(tile.view(np.uint32)[0])
    assert w0 >> 16 == 0b1100011011110000


# ---------------------------------------------------------------- codebooks

def _cb_numpy(cb: int) -> np.ndarray:
    """Codebook re-derived with numpy (codebook.cuh:57-90): uint32 wraparound arithmetic, fp16 via
    numpy's correctly rounded conversions."""
    w = np.arange(65536, dtype=np.uint64)
    if cb == 2:
        x = (w * 0x83DCD12D) & 0xFFFFFFFF
        s = (x & 0xFF) + ((x >> 8) & 0xFF) + ((x >> 16) & 0xFF) + (x >> 24)
        h = (0x6400 + s).astype(np.uint16).view(np.float16).astype(np.float64)
        c1 = np.array([0x1EEE], np.uint16).view(np.float16).astype(np.float64)[0]
        c0 = np.array([0xC931], np.uint16).view(np.float16).astype(np.float64)[0]
        return (h * c1 + c0).astype(np.float16).view(np.uint16)
    if cb == 1:
        x = (w * 0xCBAC1FED) & 0xFFFFFFFF
    else:
        x = (w * 89226354 + 64248484) & 0xFFFFFFFF
    x = (x & 0x8FFF8FFF) ^ 0x3B603B60
    lo = (x & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (x >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    return (lo + hi).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("cb", [0, 1, 2])
def test_codebook_exhaustive(cb):
    t = O.codebook_table(cb)
    assert np.array_equal(t, _cb_numpy(cb))
    sha = json.loads((GOLD / "codebook_sha256.json").read_text())
    assert hashlib.sha256(t.tobytes()).hexdigest() == sha[str(cb)]


def test_codebook2_properties():
    v = O.codebook_table(2).view(np.float16).astype(np.float64)
    c1, c0 = 0.00676727294921875, -10.3828125                    # fp16 0x1eee, 0xc931
    assert v.min() >= 1024 * c1 + c0 and v.max() <= 2044 * c1 + c0 # byte sum s in [0, 1020]
    assert v.min() == 1024 * c1 + c0                              # s = 0 (w = 0) is the minimum
    assert abs(v.mean()) < 0.01 and abs(v.std() - 1.0) < 0.01   # unit-variance Gaussian-like codebook


def test_lop3_0x6a_truth_table():
    """lop3 immediate 0x6a evaluated on the canonical operands (0xF0, 0xCC, 0xAA) is (a & b) ^ c."""
    a, b, c = 0xF0, 0xCC, 0xAA
    assert ((a & b) ^ c) == 0x6A
    assert ((a & b) | (~a & c)) & 0xFF != 0x6A


# ---------------------------------------------------------------- tile layout / reconstruct

def _tile_slot_to_index(row: int, col: int):
    """The reference's own layout model, test_reconstruct.cpp:199-211: slot (row, half2 column col)
    of a 16x16 tile holds positions (il, il + 32)."""
    b, g = col // 4, col % 4
    rb, rr = row // 8, row % 8
    r, ph = rr // 2, rr % 2
    q = ph + 2 * rb
    lane = g * 8 + r
    il = lane * 8 + q + b * 4
    return il, il + 32


@pytest.mark.parametrize("bits,cb", [(2, 2), (3, 0), (4, 1), (5, 2), (8, 0), (1, 2)])
def test_reconstruct_layout(bits, cb):
    K, N = 32, 48
    trellis, _, _ = make_linear(7 + bits, K, N, bits)
    W = O.reconstruct(trellis, K, N, bits, cb)
    table = O.codebook_table(cb)
    for tk in range(K // 16):
        for tn in range(N // 16):
            tile = trellis[tk, tn]
            win = O.unpack_tile(tile, bits)
            for k in range(16):
                for c in range(8):
                    il, ih = _tile_slot_to_index(k, c)
                    assert W[16 * tk + k, 16 * tn + 2 * c] == table[win[il]]
                    assert W[16 * tk + k, 16 * tn + 2 * c + 1] == table[win[ih]]


def test_reconstruct_golden():
    f = np.load(GOLD / "reconstruct_small.npz")
    for key in [k for k in f.files if k.startswith("trellis_")]:
        _, bits, cb = key.split("_")
        bits, cb = int(bits[1:]), int(cb[2:])
        tr = f[key]
        K, N = tr.shape[0] * 16, tr.shape[1] * 16
        assert np.array_equal(O.reconstruct(tr, K, N, bits, cb), f[f"w_b{bits}_cb{cb}"])


# ---------------------------------------------------------------- Hadamard

def test_had128_sylvester():
    H = scipy.linalg.hadamard(128).astype(np.float64) / np.sqrt(128.0)
    r = np.random.default_rng(3)
    v = r.standard_normal(256)
    got = O.had128(v)
    assert np.allclose(got[:128], H @ v[:128], rtol=0, atol=1e-12)
    assert np.allclose(got[128:], H @ v[128:], rtol=0, atol=1e-12)
    assert np.allclose(O.had128(got), v, atol=1e-12)   # H . H = I


# ---------------------------------------------------------------- linear

@pytest.mark.parametrize("bits,cb,M", [(2, 2, 1), (4, 0, 3), (3, 1, 2)])
def test_linear_matches_dense_numpy(bits, cb, M):
    """Independent dense pipeline: W_hat from reconstruct, H from scipy, fp64 matmul, with the
    reference's rounding points (x.suh fp16, a_had fp16)."""
    K, N = 256, 384
    trellis, suh, svh = make_linear(11, K, N, bits)
    x = make_x(12, M, K)
    W = O.reconstruct(trellis, K, N, bits, cb).view(np.float16).astype(np.float64)
    H = scipy.linalg.hadamard(128).astype(np.float64) / np.sqrt(128.0)
    xs = (x.astype(np.float64) * suh.astype(np.float64)).astype(np.float16).astype(np.float64)
    a = (xs.reshape(M, -1, 128) @ H.T).reshape(M, K).astype(np.float16).astype(np.float64)
    acc = a @ W
    y = (acc.reshape(M, -1, 128) @ H.T).reshape(M, N) * svh.astype(np.float64)
    got = O.linear(x, trellis, suh, svh, K, N, bits, cb)
    assert np.allclose(got, y, rtol=1e-12, atol=1e-9)


def test_linear_is_linear_in_transformed_input():
    K, N = 128, 128
    trellis, suh, svh = make_linear(5, K, N, 2)
    x1 = np.ones((1, K), np.float16)
    y1 = O.linear(x1, trellis, suh, svh, K, N, 2, 2)
    y2 = O.linear((2 * x1).astype(np.float16), trellis, suh, svh, K, N, 2, 2)
    assert np.allclose(y2, 2 * y1, rtol=1e-12)


def test_cpu_baseline_matches_oracle():
    K, N, bits = 512, 256, 2
    trellis, suh, svh = make_linear(21, K, N, bits)
    x = make_x(22, 2, K)
    ref = O.linear(x, trellis, suh, svh, K, N, bits, 2)
    got, secs = O.cpu_linear_f32(x, trellis, suh, svh, K, N, bits, 2, threads=2)
    assert secs > 0
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-4


# ---------------------------------------------------------------- router

def _route_brute(s16: np.ndarray, K: int, scale: float):
    f = s16.astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    enc = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    order = sorted(range(len(f)), key=lambda e: (-int(enc[e]), e))[:K]
    o = np.array([1.0 / (1.0 + np.exp(-float(f[e]))) for e in order])
    w = (o * scale / (o.sum() + 1e-20)).astype(np.float16)
    return np.array(order), w


def test_routing_brute_force():
    r = np.random.default_rng(9)
    s = r.standard_normal((16, 288)).astype(np.float16)
    s[3, 10] = s[3, 20] = s[3, 30] = np.float16(4.0)    # ties -> lower index first
    s[4, :] = np.float16(0.0)
    s[4, 7] = np.float16(-0.0)                          # +0 ranks above -0
    idx, w = O.routing(s, 8, 2.5)
    for b in range(16):
        bi, bw = _route_brute(s[b], 8, 2.5)
        assert np.array_equal(idx[b], bi)
        assert np.array_equal(w[b], bw.view(np.uint16))
    assert list(idx[3, :3]) == [10, 20, 30]
    assert 7 not in idx[4]
    assert np.allclose(w.view(np.float16).astype(np.float64).sum(1), 2.5, rtol=5e-3)


def _route_brute_bias(s16: np.ndarray, b16: np.ndarray, K: int, scale: float):
    """routing.cu:240-326 with a correction bias: key = fp32(sigmoid(logit)) + fp32(bias), larger
    first, ties to the lower index; the weight uses the unbiased sigmoid."""
    f = s16.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-f))
    key = (sig.astype(np.float32) + b16.astype(np.float32)).astype(np.float32)
    order = sorted(range(len(f)), key=lambda e: (-float(key[e]), e))[:K]
    o = sig[order]
    w = (o * scale / (o.sum() + 1e-20)).astype(np.float16)
    return np.array(order), w


def test_routing_bias_brute_force():
    r = np.random.default_rng(19)
    E, K = 288, 8
    s = r.standard_normal((8, E)).astype(np.float16)
    b = (r.standard_normal(E) * 0.05).astype(np.float16)
    s[2, 100] = np.float16(-6.0)
    b[100] = np.float16(4.0)       # a low logit with a large bias is selected
    idx, w = O.routing(s, K, 2.5, b)
    for row in range(8):
        bi, bw = _route_brute_bias(s[row], b, K, 2.5)
        assert np.array_equal(idx[row], bi)
        assert np.array_equal(w[row], bw.view(np.uint16))
    assert idx[2, 0] == 100
    # the weight of that expert comes from sigmoid(-6), not from the biased key
    assert w[2, 0].view(np.float16) < np.float16(0.01)
    assert not np.array_equal(idx, O.routing(s, K, 2.5)[0])


def _route_brute_general(s16, b16, K, scale, use_topk, act):
    """routing.cu:18-36 activations (sigmoid; sqrt(softplus) with threshold 20), the selection key of
    routing.cu:240-245 (use_topk) and :366-393 (sorting variant) -- act + bias with a bias, else the
    logit (use_topk) or act(logit) -- larger first, ties to the lower index; weights act(logit) over
    the selection in fp32, o * scale / sum (use_topk) or o * (scale / sum)."""
    f = s16.astype(np.float64)
    if act == 1:
        a = np.sqrt(np.where(f > 20.0, f, np.log1p(np.exp(np.minimum(f, 20.0)))))
    else:
        a = 1.0 / (1.0 + np.exp(-f))
    a32 = a.astype(np.float32)
    if b16 is not None:
        key = (a32 + b16.astype(np.float32)).astype(np.float32)
    else:
        key = f.astype(np.float32) if use_topk else a32
    order = sorted(range(len(f)), key=lambda e: (-float(key[e]), e))[:K]
    o = a32[order]
    tot = np.float32(0.0)
    for v in o:
        tot = np.float32(tot + v)
    tot = np.float32(tot + np.float32(1e-20))
    sc = np.float32(scale)
    w = (o * sc / tot) if use_topk else (o * (sc / tot))
    return np.array(order), w.astype(np.float32).astype(np.float16)


@pytest.mark.parametrize("use_topk,act,with_bias", [(1, 1, False), (1, 1, True), (0, 0, False), (0, 0, True),
                                                    (0, 1, False), (0, 1, True)])
def test_routing_variants_brute_force(use_topk, act, with_bias):
    """The router's other activation (sqrt(softplus), DSv4) and the sorting variant (use_topk=false):
    indices and weights equal a brute-force sort on the closed forms.  Logits above softplus's
    threshold 20 and a row of large logits (where the sorting variant's activated key saturates and
    ties differ from the raw-logit order) are included."""
    r = np.random.default_rng(100 + 10 * use_topk + act)
    E, K = 288, 8
    s = r.standard_normal((12, E)).astype(np.float16)
    s[1, 5] = np.float16(25.0)            # past softplus's threshold
    s[2, :] = (r.standard_normal(E) * 3 + 22).astype(np.float16)  # sigmoid saturates to 1.0f
    b = (r.standard_normal(E) * 0.05).astype(np.float16) if with_bias else None
    idx, w = O.routing(s, K, 2.5, b, use_topk=bool(use_topk), act_fn=act)
    for row in range(12):
        bi, bw = _route_brute_general(s[row], b, K, 2.5, use_topk, act)
        assert np.array_equal(idx[row], bi), row
        assert np.array_equal(w[row], bw.view(np.uint16)), row
    if not use_topk and act == 0 and not with_bias:
        # saturated sigmoid keys tie: the sorting variant takes the lowest indices of the tie,
        # the use_topk variant the largest logits
        assert not np.array_equal(idx[2], O.routing(s, K, 2.5)[0][2])


# ---------------------------------------------------------------- permutation / reduction

def test_permute_definition():
    r = np.random.default_rng(4)
    M, topk, E = 50, 8, 40
    ids = np.stack([r.permutation(E)[:topk] for _ in range(M)]).astype(np.int64)
    w = r.random((M, topk)).astype(np.float16)
    cnt, ts, ws, r2s = O.permute(ids, w, E)
    flat = ids.reshape(-1)
    assert np.array_equal(cnt[:E], np.bincount(flat, minlength=E)) and cnt[E] == 0
    order = np.argsort(flat, kind="stable")
    assert np.array_equal(ts, order // topk)
    assert np.array_equal(ws, w.reshape(-1).view(np.uint16)[order])
    assert np.array_equal(flat[order[r2s]], flat)   # route_to_sorted inverts the sort
    assert np.array_equal(r2s[order], np.arange(M * topk))


def test_reduce_sorted_reference_fixture():
    """test_deterministic_reductions.cu:49-66: terms {1e20, -1e20, 1, 1} in rank order sum to 2.0
    from +0 for every storage permutation of the contributions."""
    terms = np.array([1e20, -1e20, 1.0, 1.0], np.float32)
    import itertools
    for perm in itertools.permutations(range(4)):
        contrib = np.zeros((4, 4), np.float32)
        r2s = np.array(perm, np.int64)
        for j in range(4):
            contrib[perm[j], :] = terms[j]
        y = O.reduce_sorted(contrib, r2s, 1, 4)
        assert np.all(y == 2.0)


def test_swiglu_clamp():
    g = np.array([-20.0, -1.0, 0.0, 1.0, 12.0], np.float32)
    u = np.array([1.0, 2.0, 3.0, -15.0, 0.5], np.float32)
    out = O.swiglu_clamp(g, u, 10.0).view(np.float16).astype(np.float64)
    gv = np.minimum(g.astype(np.float64), 10.0)
    uv = np.clip(u.astype(np.float64), -10.0, 10.0)
    want = (gv / (1 + np.exp(-gv)) * uv).astype(np.float16)
    assert np.array_equal(out.astype(np.float16), want)


# ---------------------------------------------------------------- one MoE layer

def _h16(v):
    with np.errstate(over="ignore"):   # fp16 overflow to inf is part of the reference arithmetic
        return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def _silu16(g):
    """fp16 SiLU evaluated with one fp16 rounding per step: e = exp(-g), s = 1 + e, r = 1/s, g.r."""
    with np.errstate(over="ignore"):
        e = _h16(np.exp(-g))
    s = _h16(1.0 + e)
    return _h16(g * _h16(1.0 / s))


def _gelu_erf16(g):
    """x . Phi(x) (the exact GELU, scipy's erf), rounded to fp16."""
    return _h16(0.5 * g * (1.0 + scipy.special.erf(g / np.sqrt(2.0))))


def _moe_layer_numpy(x, hidden, inter, idx, wt, ex, sh, L, act=None):
    """Dense numpy restatement of one MoE layer from decoded W_hat matrices and scipy's Sylvester
    Hadamard (exl3_moe_kernel.cuh:57-262, hadamard_inner.cuh:284-481, runner.cpp:723-738,918-958);
    the routed expert is helpers.expert_contrib_numpy, which this pins.
    act: None SiLU, "gelu_erf" the exact GELU, "relu2" the non-gated relu2 (no gate GEMM)."""
    H = scipy.linalg.hadamard(128).astype(np.float64) / np.sqrt(128.0)

    def had(v):
        return (v.reshape(-1, 128) @ H.T).reshape(v.shape)

    def W(tr, K, N, bits):
        return O.reconstruct(tr, K, N, bits, 2).view(np.float16).astype(np.float64)

    def a_in(xt, suh):
        return _h16(had(_h16(xt * suh.astype(np.float64))))

    T = x.shape[0]
    xd = x.astype(np.float64)
    y_routed = np.zeros((T, hidden), np.float32)
    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
    for t in range(T):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            w_e = float(wt[t, j].view(np.float16))
            Ws = [W(ex["trellis"][p][e], *shapes[p], int(ex["bits"][p][e])) for p in range(3)]
            su = [ex["suh"][p][e].view(np.float16).astype(np.float64) for p in range(3)]
            sv = [ex["svh"][p][e].view(np.float16).astype(np.float64) for p in range(3)]
            c = expert_contrib_numpy(xd[t], *Ws, su, sv, [w_e], L, act=act)[0]
            y_routed[t] += c.astype(np.float32)   # fp32 accumulation in rank order
    y16 = None
    if sh is not None:
        def lin(v, p, K, N):
            su = sh["suh"][p].view(np.float16).astype(np.float64)
            sv = sh["svh"][p].view(np.float16).astype(np.float64)
            return had(a_in(v, su) @ W(sh["trellis"][p], K, N, int(sh["bits"][p]))) * sv
        y16 = np.empty((T, hidden), np.float16)
        for t in range(T):
            gs = np.minimum(lin(xd[t], 0, hidden, inter), L)
            us = np.clip(lin(xd[t], 1, hidden, inter), -L, L)
            act = _h16(gs / (1.0 + np.exp(-gs)) * us)
            d = lin(act, 2, inter, hidden).astype(np.float32)
            y16[t] = (y_routed[t] + d).astype(np.float16)
    return y_routed.astype(np.float64), y16


def _tiny_layer(E, hidden, inter, seed, bits=(2, 3, 2)):
    ex = {"trellis": [[], [], []], "suh": [[], [], []], "svh": [[], [], []], "bits": []}
    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
    for p, (K, N) in enumerate(shapes):
        for e in range(E):
            tr, suh, svh = make_linear(seed + 10 * e + p, K, N, bits[p])
            ex["trellis"][p].append(tr)
            ex["suh"][p].append(suh.view(np.uint16))
            ex["svh"][p].append(svh.view(np.uint16))
        ex["bits"].append(np.full(E, bits[p], np.int32))
    sh = {"trellis": [], "suh": [], "svh": [], "bits": []}
    for p, (K, N) in enumerate(shapes):
        tr, suh, svh = make_linear(seed + 1000 + p, K, N, 2)
        sh["trellis"].append(tr)
        sh["suh"].append(suh.view(np.uint16))
        sh["svh"].append(svh.view(np.uint16))
        sh["bits"].append(2)
    return ex, sh


@pytest.mark.parametrize("L", [6.0, 0.0])
def test_moe_rows_matches_dense_numpy(L):
    """hx_or_moe_rows against the dense numpy layer: same fp16 rounding points, fp64 matmuls in a
    different summation order, so values agree to an fp16 ulp or two where a rounding flips."""
    E, hidden, inter, topk, T = 4, 256, 256, 2, 3
    ex, sh = _tiny_layer(E, hidden, inter, 40)
    x = make_x(41, T, hidden)
    scores = make_x(42, T, E)
    idx, w = O.routing(scores, topk, 2.5)
    yr, yo = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), ex, sh if L else None, L)
    yr_np, yo_np = _moe_layer_numpy(x, hidden, inter, idx, w, ex, sh if L else None, L)
    scale = np.abs(yr_np).max()
    assert scale > 1.0
    assert np.abs(yr - yr_np).max() <= 2e-3 * scale
    assert np.mean(np.abs(yr - yr_np) <= 1e-6 * scale) > 0.9   # most rows bit-identical up to fp32 order
    if L:
        got = yo.view(np.float16).astype(np.float64)
        assert np.abs(got - yo_np.astype(np.float64)).max() <= 2e-3 * np.abs(yo_np.astype(np.float64)).max()
        assert np.mean(got == yo_np.astype(np.float64)) > 0.9


def test_moe_rows_weight_linearity_and_row_selection():
    """c = H(D) . w . svh_d is linear in the routing weight (a power of two scales exactly); rows
    selects tokens; an expert repeated in both ranks doubles its contribution."""
    E, hidden, inter = 3, 128, 128
    ex, _ = _tiny_layer(E, hidden, inter, 50)
    x = make_x(51, 2, hidden)
    idx = np.array([[1], [2]], np.int64)
    w1 = np.array([[1.0], [0.5]], np.float16).view(np.uint16)
    w2 = np.array([[2.0], [1.0]], np.float16).view(np.uint16)
    y1, _ = O.moe_rows(x, hidden, inter, idx, w1, np.arange(2), ex, None, 0.0)
    y2, _ = O.moe_rows(x, hidden, inter, idx, w2, np.arange(2), ex, None, 0.0)
    assert np.array_equal(y2, 2 * y1)
    y_sel, _ = O.moe_rows(x, hidden, inter, idx, w1, np.array([1]), ex, None, 0.0)
    assert np.array_equal(y_sel[0], y1[1])
    idx2 = np.array([[1, 1]], np.int64)
    w_pair = np.array([[1.0, 1.0]], np.float16).view(np.uint16)
    yp, _ = O.moe_rows(x[:1], hidden, inter, idx2, w_pair, np.arange(1), ex, None, 0.0)
    assert np.array_equal(yp[0], (2 * y1[0].astype(np.float32)).astype(np.float64))


def test_moe_rows_gelu_near_exact_gelu():
    """act 1 (tanh-form GELU): the tanh form stays within 1e-3 of x.Phi(x) (its published maximum
    deviation is about 5e-4 near |x| = 2), so the layer lands within a few fp16 ulps of the same
    layer with the exact GELU; and it differs from the SiLU layer (the activation is applied; both tend to x for large x, so
    the difference is small but well above rounding)."""
    E, hidden, inter, topk, T = 4, 256, 256, 2, 3
    ex, _ = _tiny_layer(E, hidden, inter, 60)
    x = make_x(61, T, hidden)
    idx, w = O.routing(make_x(62, T, E), topk, 2.5)
    yr, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), ex, None, 6.0, act=1)
    y_erf, _ = _moe_layer_numpy(x, hidden, inter, idx, w, ex, None, 6.0, act="gelu_erf")
    y_silu, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), ex, None, 6.0, act=0)
    scale = np.abs(y_erf).max()
    assert scale > 1.0
    assert np.abs(yr - y_erf).max() <= 1e-2 * scale
    assert np.abs(yr - y_silu).max() > 0.01 * scale


@pytest.mark.parametrize("L", [6.0, 0.0])
def test_moe_rows_relu2_nogate(L):
    """act 2 (non-gated relu2): the gate projection is never read (garbage gate weights change
    nothing), the activation is relu(u) . clamp(u) -- matched by the dense numpy layer -- and,
    with no limit, halving x quarters the down input before rounding (degree-2 homogeneity,
    checked on the layer within fp16 rounding)."""
    E, hidden, inter, topk, T = 4, 256, 256, 2, 3
    ex, _ = _tiny_layer(E, hidden, inter, 70)
    x = make_x(71, T, hidden)
    idx, w = O.routing(make_x(72, T, E), topk, 2.5)
    yr, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), ex, None, L, act=2)
    junk = {k: [list(v) for v in ex[k]] if k != "bits" else list(ex[k]) for k in ex}
    rng = np.random.default_rng(73)
    junk["trellis"][0] = [rng.integers(0, 65536, t.shape, dtype=np.uint16) for t in ex["trellis"][0]]
    junk["suh"][0] = [np.full_like(a, 0x7C00) for a in ex["suh"][0]]   # +inf: would poison any read
    junk["svh"][0] = [np.full_like(a, 0x7C00) for a in ex["svh"][0]]
    yj, _ = O.moe_rows(x, hidden, inter, idx, w, np.arange(T), junk, None, L, act=2)
    assert np.array_equal(yr, yj)
    y_np, _ = _moe_layer_numpy(x, hidden, inter, idx, w, ex, None, L, act="relu2")
    scale = np.abs(y_np).max()
    assert scale > 1.0
    assert np.abs(yr - y_np).max() <= 2e-3 * scale
    if not L:
        xh = (x.view(np.float16) * np.float16(0.5)).view(np.uint16)
        yh, _ = O.moe_rows(xh, hidden, inter, idx, w, np.arange(T), ex, None, 0.0, act=2)
        assert np.abs(4 * yh - yr).max() <= 2e-2 * scale


def test_h128_register_sign_pattern():
    """The sign rule the matrix-core Hadamard kernels use to build H128 B operands in registers: for
    n = 16 nb + c and k = 32 kk + 8 g + j (c < 16, g < 4, j < 8), popcount(n & k) is odd exactly when
    popcount(c & j & 7) + (c3 & g0) + (nb0 & g1) + (nb1 & kk0) + (nb2 & kk1) is odd -- checked against
    scipy's Sylvester matrix over all 128 x 128 entries."""
    H = scipy.linalg.hadamard(128)
    for n in range(128):
        nb, c = n >> 4, n & 15
        for k in range(128):
            kk, g, j = k >> 5, (k >> 3) & 3, k & 7
            par = (bin(c & j & 7).count("1") + ((c >> 3) & g & 1) + ((nb & 1) & (g >> 1)) + ((nb >> 1) & kk & 1)
                   + ((nb >> 2) & (kk >> 1) & 1)) & 1
            assert H[k, n] == (-1 if par else 1)


def test_pack_signs_oracle():
    """pack_signs: the reference kernel's shift-in loop puts value i's sign in bit i.  Pinned by a
    worked example of that loop (only the first value negative -> 0x0001, only the last -> 0x8000,
    alternating signs starting negative -> 0x5555) and, for random columns, by the bit-position formula
    sum_i sign_i << i computed independently with numpy."""
    def col(signs):
        return np.array([0xbc00 if s else 0x3c00 for s in signs], np.uint16)  # -1.0 / +1.0
    assert O.pack_signs(col([1] + [0] * 15), 1)[0] == 0x0001
    assert O.pack_signs(col([0] * 15 + [1]), 1)[0] == 0x8000
    assert O.pack_signs(col([1, 0] * 8), 1)[0] == 0x5555
    r = np.random.default_rng(5)
    u = r.integers(0, 65536, size=(300, 16), dtype=np.uint16)
    want = ((u >> 15).astype(np.uint32) << np.arange(16, dtype=np.uint32)).sum(axis=1).astype(np.uint16)
    assert np.array_equal(O.pack_signs(u.reshape(-1), 300), want)


def test_count_inf_nan_oracle():
    """count_inf_nan: every fp16 bit pattern against numpy's isinf/isnan, fp32 specials, and the
    reference test's known answer (test_reconstruct.cpp:468-493: 4096 values of 0.5 with +inf at 17,
    -inf at 900 and a NaN at 2000 give inf = 2, nan = 1)."""
    allh = np.arange(65536, dtype=np.uint16)
    f = allh.view(np.float16)
    assert O.count_inf_nan(allh) == (int(np.isinf(f).sum()), int(np.isnan(f).sum())) == (2, 2046)
    kat = np.full(4096, 0x3800, np.uint16)
    kat[17], kat[900], kat[2000] = 0x7c00, 0xfc00, 0x7e00
    assert O.count_inf_nan(kat) == (2, 1)
    f32 = np.array([1.0, np.inf, -np.inf, np.nan, -np.nan, 3.4e38, 0.0], np.float32)
    assert O.count_inf_nan(f32) == (2, 2)
