"""Checkpoint loader: safetensors shards -> expert slab / GroupWords (names, shapes, dtypes, mul1 checks
of src/core/expert_layout.cpp:6-55 and model.cpp:74-90), bit-exact placement, and a layer loaded from
a file against the CPU oracle."""
import numpy as np
import pytest

from helpers import assert_close

safetensors_numpy = pytest.importorskip("safetensors.numpy")

MUL1_I32 = np.int32(0x83DCD12D - (1 << 32))
PREFIX = "model.language_model.layers"


def _linear(r, K, N, bits):
    tr = r.integers(-32768, 32768, size=(K // 16, N // 16, 16 * bits), dtype=np.int16)
    suh = r.choice([-1.0, 1.0], K).astype(np.float16)
    svh = (r.choice([-1.0, 1.0], N) * r.uniform(0.5, 1.5, N)).astype(np.float16)
    return tr, suh, svh


def make_checkpoint(path, E=3, hidden=256, inter=128, bits=((2, 2, 2), (3, 2, 4), (2, 3, 2)), shared=(2, 2, 2),
                    layer=0, seed=0, shards=2):
    """A synthetic checkpoint of one MoE layer (routed experts + shared expert) split over shards;
    returns the arrays written, keyed by tensor name."""
    r = np.random.default_rng(seed)
    tensors = {}
    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
    groups = [(f"{PREFIX}.{layer}.mlp.experts.{e}", bits[e]) for e in range(E)]
    if shared:
        groups.append((f"{PREFIX}.{layer}.mlp.shared_experts", shared))
    for base, bb in groups:
        for pn, (K, N), b in zip(("gate_proj", "up_proj", "down_proj"), shapes, bb):
            tr, suh, svh = _linear(r, K, N, b)
            tensors[f"{base}.{pn}.trellis"] = tr
            tensors[f"{base}.{pn}.suh"] = suh
            tensors[f"{base}.{pn}.svh"] = svh
            tensors[f"{base}.{pn}.mul1"] = np.array(MUL1_I32, dtype=np.int32)
    names = sorted(tensors)
    for s in range(shards):
        part = {n: tensors[n] for n in names[s::shards]}
        safetensors_numpy.save_file(part, str(path / f"model-{s:05d}-of-{shards:05d}.safetensors"))
    return tensors


def test_shardset_reads_every_tensor(tmp_path):
    from helios_glm53flash_amd import checkpoint as ck
    tensors = make_checkpoint(tmp_path)
    ss = ck.ShardSet(tmp_path)
    assert len(ss.paths) == 2 and set(ss.tensors) == set(tensors)
    for name, arr in tensors.items():
        got = ss.read(ss.find(name))
        assert got.dtype == arr.dtype and got.shape == arr.shape and np.array_equal(got, arr), name
    assert ss.find("nope") is None


def test_expert_slab_layout_and_bytes(tmp_path):
    from helios_glm53flash_amd import checkpoint as ck
    tensors = make_checkpoint(tmp_path)
    ss = ck.ShardSet(tmp_path)
    lay, _ = ck.expert_layout(ss, 0, 3, 256, 128)
    starts = [o for e in lay.off for p in e for o in p]
    assert all(o % ck.PIECE_ALIGN == 0 for o in starts) and len(set(starts)) == len(starts)
    assert lay.bits == [[2, 2, 2], [3, 2, 4], [2, 3, 2]]
    ex = ck.load_experts(ss, 0, 3, 256, 128, device="cpu")
    assert ex.bits == [[2, 3, 2], [2, 2, 3], [2, 4, 2]]  # [projection][expert]
    for e in range(3):
        for p, pn in enumerate(("gate_proj", "up_proj", "down_proj")):
            base = f"{PREFIX}.0.mlp.experts.{e}.{pn}"
            assert np.array_equal(ex.trellis[p][e].numpy(), tensors[base + ".trellis"])
            assert np.array_equal(ex.suh[p][e].numpy(), tensors[base + ".suh"])
            assert np.array_equal(ex.svh[p][e].numpy(), tensors[base + ".svh"])
    sh = ck.load_shared_mlp(ss, 0, 256, 128, device="cpu")
    assert [g.bits for g in sh] == [2, 2, 2] and sh[0].mul1 == 0x83DCD12D
    assert ck.load_shared_mlp(ss, 1, 256, 128, device="cpu") is None


@pytest.mark.parametrize("defect", ["missing", "mul1", "shape", "dtype", "suh_len"])
def test_expert_validation_names_the_tensor(tmp_path, defect):
    from helios_glm53flash_amd import checkpoint as ck
    tensors = make_checkpoint(tmp_path, shards=1)
    bad = f"{PREFIX}.0.mlp.experts.1.up_proj"
    if defect == "missing":
        del tensors[bad + ".svh"]
    elif defect == "mul1":
        tensors[bad + ".mul1"] = np.array(12345, dtype=np.int32)
    elif defect == "shape":
        tensors[bad + ".trellis"] = tensors[bad + ".trellis"][:, :4].copy()
    elif defect == "dtype":
        tensors[bad + ".suh"] = tensors[bad + ".suh"].astype(np.float32)
    else:
        tensors[bad + ".suh"] = tensors[bad + ".suh"][:128].copy()
    for f in tmp_path.glob("*.safetensors"):
        f.unlink()
    safetensors_numpy.save_file(tensors, str(tmp_path / "model.safetensors"))
    ss = ck.ShardSet(tmp_path)
    with pytest.raises(ck.CheckpointError, match="experts.1.up_proj"):
        ck.expert_layout(ss, 0, 3, 256, 128)


def test_truncated_shard_is_rejected(tmp_path):
    from helios_glm53flash_amd import checkpoint as ck
    make_checkpoint(tmp_path, shards=1)
    f = next(tmp_path.glob("*.safetensors"))
    data = f.read_bytes()
    f.write_bytes(data[:-100])
    with pytest.raises(ck.CheckpointError):
        ck.ShardSet(tmp_path)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [1, 24])
def test_layer_from_checkpoint_matches_oracle(tmp_path, T):
    """Routed + shared experts loaded from safetensors into HBM; decode (T=1) and prefill (T=24) layer
    outputs against the oracle on the arrays that were written."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from helios_glm53flash_amd import checkpoint as ck, moe
    from oracle import oracle as O
    E, hidden, inter, topk = 6, 256, 128, 2
    bits = [(2, 2, 2), (3, 2, 4), (2, 3, 2), (2, 2, 2), (4, 4, 3), (2, 2, 2)]
    tensors = make_checkpoint(tmp_path, E=E, hidden=hidden, inter=inter, bits=bits, seed=7)
    ss = ck.ShardSet(tmp_path)
    ex = ck.load_experts(ss, 0, E, hidden, inter)
    sh = ck.load_shared_mlp(ss, 0, hidden, inter)
    layer = moe.MoeLayer(ex, sh, topk=topk)
    r = np.random.default_rng(T)
    x = r.standard_normal((T, hidden)).astype(np.float16)
    scores = r.standard_normal((T, E)).astype(np.float16)
    y_routed = torch.empty((T, hidden), dtype=torch.float32, device="cuda")
    y = layer(torch.from_numpy(x).cuda(), torch.from_numpy(scores).cuda(), y_routed=y_routed)
    torch.cuda.synchronize()

    def g(base, p):
        pn = ("gate_proj", "up_proj", "down_proj")[p]
        return [tensors[f"{base}.{pn}.{s}"] for s in ("trellis", "suh", "svh")]

    exp = {"trellis": [], "suh": [], "svh": [], "bits": []}
    for p in range(3):
        gs = [g(f"{PREFIX}.0.mlp.experts.{e}", p) for e in range(E)]
        exp["trellis"].append([a[0].view(np.uint16) for a in gs])
        exp["suh"].append([a[1].view(np.uint16) for a in gs])
        exp["svh"].append([a[2].view(np.uint16) for a in gs])
        exp["bits"].append(np.array([b[p] for b in bits], np.int32))
    shd = {"trellis": [], "suh": [], "svh": [], "bits": []}
    for p in range(3):
        a = g(f"{PREFIX}.0.mlp.shared_experts", p)
        shd["trellis"].append(a[0].view(np.uint16))
        shd["suh"].append(a[1].view(np.uint16))
        shd["svh"].append(a[2].view(np.uint16))
        shd["bits"].append(a[0].shape[2] // 16)
    idx, w = O.routing(scores, topk, 2.5)
    rows = np.arange(T)
    yr_ref, yo_ref = O.moe_rows(x, hidden, inter, idx, w, rows, exp, shd, 10.0)
    assert_close(y_routed.cpu().numpy(), yr_ref, what=f"routed from checkpoint T={T}")
    assert_close(y.float().cpu().numpy(), yo_ref.view(np.float16).astype(np.float64), what=f"y from checkpoint T={T}")


def test_router_bias_is_centred_and_gate_converted(tmp_path):
    """model.cpp:185-196,524-535: gate weight to fp16; bias fp32 minus its mean (fp64 sum), to fp16."""
    from helios_glm53flash_amd import checkpoint as ck
    r = np.random.default_rng(3)
    E, H = 12, 64
    gate = r.standard_normal((E, H)).astype(np.float32)
    bias = (r.standard_normal(E) * 3 + 7).astype(np.float32)
    bf16 = (gate.view(np.uint32) >> 16).astype(np.uint16)  # truncated bf16 bits of the gate
    safetensors_numpy.save_file({f"{PREFIX}.2.mlp.gate.weight": gate,
                                 f"{PREFIX}.2.mlp.gate.e_score_correction_bias": bias}, str(tmp_path / "a.safetensors"))
    w, b = ck.load_router(ck.ShardSet(tmp_path), 2, E, H, device="cpu")
    assert np.array_equal(w.numpy(), gate.astype(np.float16))
    mean = np.float32(bias.astype(np.float64).sum() / E)
    assert np.array_equal(b.numpy(), (bias - mean).astype(np.float16))
    assert abs(float(b.float().mean())) < 1e-2
    (tmp_path / "a.safetensors").unlink()
    import json, struct
    hdr = json.dumps({f"{PREFIX}.2.mlp.gate.weight": {"dtype": "BF16", "shape": [E, H],
                                                      "data_offsets": [0, E * H * 2]}}).encode()
    (tmp_path / "b.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bf16.tobytes())
    w, b = ck.load_router(ck.ShardSet(tmp_path), 2, E, H, device="cpu")
    assert b is None
    assert np.array_equal(w.numpy(), (bf16.astype(np.uint32) << 16).view(np.float32).astype(np.float16))
    assert ck.load_router(ck.ShardSet(tmp_path), 3, E, H, device="cpu") == (None, None)


# ---------------------------------------------------------------- the native (C++) loader

def _ref_layout(pieces):
    """expert_layout.cpp:48-52: pieces in order, each projection's end rounded up to 64 bytes."""
    off, pos = [], 0
    for q, n in enumerate(pieces):
        off.append(pos)
        pos += n
        if q % 4 == 3:
            pos = (pos + 63) & ~63
    return off, pos


def test_native_layout_follows_the_reference(tmp_path):
    """hx_ckpt_open / hx_ckpt_expert_layout (C++, host only): every tensor found across the shards,
    the bit widths, piece sizes and offsets of expert_layout.cpp, and the index file's shard list."""
    from helios_glm53flash_amd import checkpoint as ck
    E, hidden, inter = 3, 256, 128
    tensors = make_checkpoint(tmp_path, E=E, hidden=hidden, inter=inter, bits=((2, 3, 4),) * E)
    nc = ck.NativeCheckpoint(tmp_path)
    assert nc.tensor_count() == len(tensors)
    lay = nc.expert_layout(0, E, hidden, inter)
    assert list(lay.bits) == [2, 3, 4]
    pieces = []
    for p, (K, N) in enumerate([(hidden, inter), (hidden, inter), (inter, hidden)]):
        pieces += [K * N * lay.bits[p] // 8, 2 * K, 2 * N, 4]
    off, stride = _ref_layout(pieces)
    assert list(lay.piece) == pieces and list(lay.off) == off and lay.stride == stride
    # an index file names the shards: an extra, unlisted shard is not read
    import json
    names = sorted(p.name for p in tmp_path.glob("*.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": names[0]}}))
    assert ck.NativeCheckpoint(tmp_path).tensor_count() < len(tensors)


@pytest.mark.parametrize("defect", ["missing", "mul1", "shape", "dtype", "suh_len", "mixed"])
def test_native_validation_names_the_tensor(tmp_path, defect):
    from helios_glm53flash_amd import checkpoint as ck
    from helios_glm53flash_amd._lib import HxError
    tensors = make_checkpoint(tmp_path, shards=1, bits=((2, 2, 2),) * 3)
    bad = f"{PREFIX}.0.mlp.experts.1.up_proj"
    if defect == "missing":
        del tensors[bad + ".svh"]
    elif defect == "mul1":
        tensors[bad + ".mul1"] = np.array(12345, dtype=np.int32)
    elif defect == "shape":
        tensors[bad + ".trellis"] = tensors[bad + ".trellis"][:, :4].copy()
    elif defect == "dtype":
        tensors[bad + ".suh"] = tensors[bad + ".suh"].astype(np.float32)
    elif defect == "suh_len":
        tensors[bad + ".suh"] = tensors[bad + ".suh"][:128].copy()
    else:  # another width than expert 0's: the reference's layout has one width per projection
        tensors[bad + ".trellis"] = np.zeros((256 // 16, 128 // 16, 48), np.int16)
    for f in tmp_path.glob("*.safetensors"):
        f.unlink()
    safetensors_numpy.save_file(tensors, str(tmp_path / "model.safetensors"))
    nc = ck.NativeCheckpoint(tmp_path)
    with pytest.raises(HxError, match="experts.1.up_proj"):
        nc.expert_layout(0, 3, 256, 128)


def test_native_rejects_truncated_shard(tmp_path):
    from helios_glm53flash_amd import checkpoint as ck
    from helios_glm53flash_amd._lib import HxError
    make_checkpoint(tmp_path, shards=1)
    f = next(tmp_path.glob("*.safetensors"))
    f.write_bytes(f.read_bytes()[:-100])
    with pytest.raises(HxError, match="data range"):
        ck.NativeCheckpoint(tmp_path)


@pytest.mark.gpu
def test_native_load_experts_and_layer(tmp_path):
    """hx_ckpt_load_experts + hx_ckpt_expert_tables: the slab holds every expert's bytes at the
    layout's offsets, and a layer run on the native tables equals the same layer on the Python
    loader's (bit for bit)."""
    import torch
    from helios_glm53flash_amd import checkpoint as ck
    from helios_glm53flash_amd import moe
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    E, hidden, inter = 6, 512, 256
    tensors = make_checkpoint(tmp_path, E=E, hidden=hidden, inter=inter, bits=((2, 2, 3),) * E, shared=None, shards=3)
    nat = ck.NativeCheckpoint(tmp_path).load_experts(0, E, hidden, inter)
    py = ck.load_experts(ck.ShardSet(tmp_path), 0, E, hidden, inter)
    for e in range(E):
        for p, pn in enumerate(("gate_proj", "up_proj", "down_proj")):
            base = f"{PREFIX}.0.mlp.experts.{e}.{pn}"
            assert np.array_equal(nat.trellis[p][e].cpu().numpy(), tensors[base + ".trellis"])
            assert np.array_equal(nat.suh[p][e].cpu().numpy(), tensors[base + ".suh"])
            assert np.array_equal(nat.svh[p][e].cpu().numpy(), tensors[base + ".svh"])
    r = np.random.default_rng(1)
    for T in (1, 20):
        x = torch.from_numpy(r.standard_normal((T, hidden)).astype(np.float16)).cuda()
        s = torch.from_numpy(r.standard_normal((T, E)).astype(np.float16)).cuda()
        ya = moe.MoeLayer(nat, None, topk=2)(x, s)
        yb = moe.MoeLayer(py, None, topk=2)(x, s)
        torch.cuda.synchronize()
        assert torch.equal(ya, yb), T


def test_native_rejects_shard_outside_directory(tmp_path):
    """An index whose weight map names '../x' or an absolute path is refused, not followed."""
    import json
    from helios_glm53flash_amd import checkpoint as ck
    from helios_glm53flash_amd._lib import HxError
    make_checkpoint(tmp_path, shards=1)
    for bad in ("../outside.safetensors", "/etc/passwd", "sub/inner.safetensors"):
        (tmp_path / "model.safetensors.index.json").write_text(json.dumps({"weight_map": {"a": bad}}))
        with pytest.raises(HxError, match="outside the checkpoint directory"):
            ck.NativeCheckpoint(tmp_path)


@pytest.mark.parametrize("offsets", ["[0, 12-3]", "[+0, 4]", "[0, 4e0]", "[0, 99999999999999999999999]", "[0, 4.]"])
def test_native_rejects_malformed_offsets(tmp_path, offsets):
    """data_offsets must be plain JSON integers: '12-3', '+0', '4e0', an overflowing integer or '4.' are
    header errors, not numbers read up to the first odd character."""
    import struct
    from helios_glm53flash_amd import checkpoint as ck
    from helios_glm53flash_amd._lib import HxError
    head = ('{"t": {"dtype": "F16", "shape": [2], "data_offsets": %s}}' % offsets).encode()
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(head)) + head + b"\0" * 16)
    with pytest.raises(HxError):
        ck.NativeCheckpoint(tmp_path)


def test_native_accepts_plain_offsets(tmp_path):
    import struct
    from helios_glm53flash_amd import checkpoint as ck
    head = b'{"__metadata__": {"v": -1.5e+2}, "t": {"dtype": "F16", "shape": [2], "data_offsets": [0, 4]}}'
    (tmp_path / "model.safetensors").write_bytes(struct.pack("<Q", len(head)) + head + b"\0" * 4)
    assert ck.NativeCheckpoint(tmp_path).tensor_count() == 1
