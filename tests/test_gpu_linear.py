"""Parity of the HIP EXL3 path (through the C ABI) against the CPU oracle."""
import numpy as np
import pytest

from helpers import assert_close, make_linear, make_x

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


@pytest.mark.parametrize("bits", range(1, 9))
@pytest.mark.parametrize("cb", [0, 1, 2])
def test_reconstruct_bit_exact_golden(hx, bits, cb):
    import torch
    from pathlib import Path
    f = np.load(Path(__file__).parent / "golden" / "reconstruct_small.npz")
    tr = f[f"trellis_b{bits}_cb{cb}"]
    want = f[f"w_b{bits}_cb{cb}"]
    K, N = tr.shape[0] * 16, tr.shape[1] * 16
    out = torch.empty((K, N), dtype=torch.float16, device="cuda")
    hx.reconstruct(out, _dev(tr, torch.int16), K // 16, N // 16, N, bits, cb == 1, cb == 2)
    torch.cuda.synchronize()
    got = out.cpu().view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)


def test_reconstruct_slice_offset(hx):
    import torch
    from oracle import oracle as O
    K, N, bits = 64, 512, 3
    tr, _, _ = make_linear(3, K, N, bits)
    want = O.reconstruct(tr, K, N, bits, 2)[:, 256:384]
    out = torch.empty((K, 128), dtype=torch.float16, device="cuda")
    hx.reconstruct_slice(out, _dev(tr, torch.int16), K // 16, N // 16, 128, bits, False, True, 256)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().view(torch.int16).numpy().view(np.uint16), want)


def _run_linear(hx, M, K, N, bits, cb, y_fp32, seed=0):
    import torch
    from oracle import oracle as O
    tr, suh, svh = make_linear(seed + 1, K, N, bits)
    x = make_x(seed + 2, M, K)
    w = hx.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), hx.MUL1 if cb == 2 else 0)
    y = torch.empty((M, N), dtype=torch.float32 if y_fp32 else torch.float16, device="cuda")
    path = hx.gemm(y, _dev(x), w, M, N, K, bits, y_fp32, mcg=(cb == 1))
    torch.cuda.synchronize()
    ref = O.linear(x, tr, suh, svh, K, N, bits, cb, out_f16=not y_fp32)
    return path, y.float().cpu().numpy(), ref


@pytest.mark.parametrize("M", [1, 3, 8, 13, 16])
@pytest.mark.parametrize("bits,cb", [(2, 2), (3, 2), (4, 2), (4, 0), (5, 1), (6, 2), (8, 2), (1, 0), (7, 1)])
def test_gemv_parity(hx, M, bits, cb):
    path, got, ref = _run_linear(hx, M, 1024, 512, bits, cb, True, seed=M * 10 + bits)
    assert path == hx.HX_GEMM_PATH_GEMV
    assert_close(got, ref, what=f"gemv M={M} bits={bits} cb={cb}")


def test_gemv_fp16_out_and_repeat(hx):
    # second call reuses the workspace counters (must have been reset by the first)
    for _ in range(3):
        _, got, ref = _run_linear(hx, 2, 2048, 1024, 2, 2, False, seed=5)
        assert_close(got, ref, what="gemv fp16 out")


def test_gemv_attention_projection_shape(hx):
    """K=4096 -> N=12288, 4-bit, M in {1, 4, 8}."""
    for M in (1, 8):
        _, got, ref = _run_linear(hx, M, 4096, 12288, 4, 2, True, seed=40 + M)
        assert_close(got, ref, what=f"attn proj M={M}")


@pytest.mark.parametrize("M", [17, 32, 100, 256])
@pytest.mark.parametrize("bits,cb", [(2, 2), (3, 2), (4, 0), (5, 2)])
def test_mfma_parity(hx, M, bits, cb):
    path, got, ref = _run_linear(hx, M, 512, 384, bits, cb, True, seed=M + bits)
    assert path == hx.HX_GEMM_PATH_MFMA
    assert_close(got, ref, what=f"mfma M={M} bits={bits} cb={cb}")


def test_mfma_fp16_out(hx):
    _, got, ref = _run_linear(hx, 64, 1024, 256, 2, 2, False, seed=77)
    assert_close(got, ref, what="mfma fp16")


def test_config1_single_linear(hx):
    """K=4096, N=2048, 2-bit, M=1 vs fp64 decode+matmul."""
    _, got, ref = _run_linear(hx, 1, 4096, 2048, 2, 2, True, seed=1)
    assert_close(got, ref, what="config 1")


@pytest.mark.parametrize("M", [1, 64])
def test_dense_3bit_real_shape(hx, M):
    """3-bit dense linear at a projection's real shape (K=4096 -> N=12288), GEMV and MFMA paths."""
    path, got, ref = _run_linear(hx, M, 4096, 12288, 3, 2, True, seed=300 + M)
    assert path == (hx.HX_GEMM_PATH_GEMV if M <= 16 else hx.HX_GEMM_PATH_MFMA)
    assert_close(got, ref, what=f"3-bit 4096x12288 M={M}")


@pytest.mark.parametrize("cb", [2, 1, 0])
def test_gemv_stream_k_sampled_columns(hx, cb):
    """One row whose split-K grid would be one workgroup per column group, unevenly spread over the
    256 CUs (1100 groups), takes the stream-K grid: 1024 workgroups over equal runs of (column group,
    128-k block) units, so most column groups are shared by two workgroups whose partials the last
    arriver adds.  Sampled column groups against the oracle, fp16 output, three calls in a row (the
    arrival counters are reset by each call, and the result is the same every time); codebooks mul1
    (2), MCG (1) and the 3INST table (0)."""
    import torch
    from oracle import oracle as O
    K, N, bits = 4096, 1100 * 128, 2
    tr, suh, svh = make_linear(702 + cb, K, N, bits)
    x = make_x(703, 1, K)
    w = hx.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), hx.MUL1 if cb == 2 else 0)
    # workgroup i takes units [i*T/1024, (i+1)*T/1024) of T = 1100 * 32 (34.4 blocks each): groups 1,
    # 30, 31 and 32 are split over two workgroups, 0, 549, 550 and the last lie in one
    groups = (0, 1, 30, 31, 32, 549, 550, N // 128 - 1)
    refs = {}
    for g in groups:
        sl = slice(128 * g, 128 * g + 128)
        sub = np.ascontiguousarray(tr[:, 8 * g:8 * g + 8, :])
        refs[g] = O.linear(x, sub, suh, np.ascontiguousarray(svh[sl]), K, 128, bits, cb, out_f16=True)
    first = None
    for call in range(3):
        y = torch.empty((1, N), dtype=torch.float16, device="cuda")
        assert hx.gemm(y, _dev(x), w, 1, N, K, bits, False, mcg=(cb == 1)) == hx.HX_GEMM_PATH_GEMV
        torch.cuda.synchronize()
        got = y.float().cpu().numpy()
        for g in groups:
            sl = slice(128 * g, 128 * g + 128)
            assert_close(got[:, sl], refs[g], what=f"stream-K {bits}-bit cb {cb} group {g} call {call}")
        if first is None:
            first = got
        else:
            assert np.array_equal(got, first), "stream-K result changed between calls"


@pytest.mark.parametrize("M", [1, 512])
def test_lm_head_6bit_sampled_columns(hx, M):
    """6-bit lm_head at its real shape (K=4096 -> N=151552), GEMV (M=1) and MFMA (M=512) paths; the
    oracle checks sampled 128-column groups (each group's output transform is independent of the
    others, so a tile-column slice of the weight is an exact sub-problem)."""
    import torch
    from oracle import oracle as O
    K, N, bits = 4096, 151552, 6
    tr, suh, svh = make_linear(600 + M, K, N, bits)
    x = make_x(601 + M, M, K)
    w = hx.GroupWords(_dev(tr, torch.int16), _dev(suh), _dev(svh), hx.MUL1)
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    a_had = torch.empty((M, K), dtype=torch.float16, device="cuda") if M > hx.GEMV_MAX_M else None
    hx.gemm(y, _dev(x), w, M, N, K, bits, True, a_had=a_had)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    rows = np.arange(M) if M <= 16 else np.array([0, 1, 255, 256, 511])
    for g in (0, 517, N // 128 - 1):
        sl = slice(128 * g, 128 * g + 128)
        sub = np.ascontiguousarray(tr[:, 8 * g:8 * g + 8, :])
        ref = O.linear(x[rows], sub, suh, np.ascontiguousarray(svh[sl]), K, 128, bits, 2, out_f16=False)
        assert_close(got[rows, sl], ref, what=f"lm_head 6-bit M={M} group {g}")


@pytest.mark.parametrize("K", range(1, 9))
def test_pack_unpack_trellis_bit_exact(hx, K):
    """pack_trellis / unpack_trellis (pack.cu): GPU packing equals the oracle's packer for every block,
    and unpacking returns the symbols (low K bits of the oracle's windows)."""
    import torch
    from oracle import oracle as O
    rows, cols = 3, 5
    r = np.random.default_rng(K)
    sym = r.integers(0, 65536, size=(rows * cols, 256), dtype=np.uint16)  # bits above K are ignored
    packed = torch.empty((rows * cols, 16 * K), dtype=torch.int16, device="cuda")
    hx.pack_trellis(packed, _dev(sym, torch.int16), rows, cols, K)
    back = torch.empty((rows * cols, 256), dtype=torch.int16, device="cuda")
    hx.unpack_trellis(back, packed, rows, cols, K)
    torch.cuda.synchronize()
    got = packed.cpu().numpy().view(np.uint16)
    mask = (1 << K) - 1
    for b in range(rows * cols):
        want = O.pack_tile(sym[b] & mask, K)
        assert np.array_equal(got[b], want), b
        assert np.array_equal(O.unpack_tile(want, K) & mask, sym[b] & mask)
    assert np.array_equal(back.cpu().numpy().view(np.uint16), sym & mask)


@pytest.mark.parametrize("bits,cb", [(2, 2), (3, 0), (4, 1), (6, 2)])
def test_reconstruct_had_slice(hx, bits, cb):
    """Original-basis weights diag(suh) H W_hat H diag(svh) / 128 per 128 x 128 tile against fp64 on the
    bit-exact W_hat; a column slice with its pre-offset svh."""
    import torch
    from oracle import oracle as O
    K, N = 256, 512
    tr, suh, svh = make_linear(90 + bits, K, N, bits)
    w_hat = O.reconstruct(tr, K, N, bits, cb).view(np.float16).astype(np.float64)
    idx = np.arange(128)
    H = np.where(np.array([[bin(i & j).count("1") & 1 for j in idx] for i in idx]) == 0, 1.0, -1.0)
    ref = np.empty((K, N))
    for a in range(0, K, 128):
        for b in range(0, N, 128):
            ref[a:a + 128, b:b + 128] = H @ w_hat[a:a + 128, b:b + 128] @ H / 128.0
    ref *= suh.astype(np.float64)[:, None] * svh.astype(np.float64)[None, :]
    out = torch.empty((K, N), dtype=torch.float16, device="cuda")
    hx.reconstruct_had_slice(out, _dev(tr, torch.int16), _dev(suh), _dev(svh), K // 16, N // 16, K, N, bits,
                             cb == 1, cb == 2, 0)
    part = torch.empty((K, 256), dtype=torch.float16, device="cuda")
    hx.reconstruct_had_slice(part, _dev(tr, torch.int16), _dev(suh), _dev(np.ascontiguousarray(svh[128:384])),
                             K // 16, N // 16, K, 256, bits, cb == 1, cb == 2, 128)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), ref, what=f"reconstruct_had bits={bits} cb={cb}")
    assert np.array_equal(part.cpu().numpy(), out.cpu().numpy()[:, 128:384])
