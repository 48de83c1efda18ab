"""Benchmark of the EXL3 MoE hot path on one MI355X.

Headline (BASELINE.json metric): weight GB/s of the MoE decode layer (config 3: 288 routed experts
+ 1 shared, 4096 -> 2048 -> 4096, 2-bit EXL3 (mul1 codebook), top-8 sigmoid router, 1 token),
counting compressed EXL3 bytes (trellis + suh + svh) of the 8 routed experts and the shared expert
read per step.  A step is one full layer: router top-k, permutation, gate/up, SiLU-gate, down,
ordered reduction and shared-expert combine.  Weights are resident in HBM; steps rotate over
independent layers (distinct weights, independent seeded router scores) so consecutive steps do not
hit the 256 MB MALL with the previous step's experts.

Also reported (extra): prefill expert-GEMM TFLOP/s (config 4: 4096 tokens, Zipf(1.1) routing, half
2-bit / half 3-bit experts), the per-phase split, and the CPU baseline (the C oracle's fp32 decode +
GEMV over the same experts, OpenMP, on this host).

python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

METRIC = "EXL3 MoE decode weight GB/s (% of HBM peak) + prefill expert-GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0


def zipf_scores(T: int, E: int, s: float, seed: int) -> np.ndarray:
    """log(Zipf(s) popularity of a seeded expert permutation) + Gumbel noise -> fp16 logits."""
    r = np.random.default_rng(seed)
    perm = r.permutation(E)
    pop = np.empty(E)
    pop[perm] = np.arange(1, E + 1, dtype=np.float64) ** (-s)
    logits = np.log(pop)[None, :] + r.gumbel(size=(T, E))
    return logits.astype(np.float16)


def bench_decode(args, torch, moe, lib):
    E, hidden, inter, topk, bits = 288, 4096, 2048, 8, 2
    L = args.layers
    layers = []
    for li in range(L):
        ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=1000 + li)
        sh = moe.synthetic_dense_mlp(hidden, inter, bits, seed=5000 + li)
        layers.append(moe.MoeLayer(ex, sh, topk=topk))
    nsteps = args.warmup + args.steps
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    # one score row per step, and at least one per rotating layer (the graph below holds one step of each)
    nrows = max(nsteps, L)
    scores = torch.randn((nrows, 1, E), generator=g, device="cuda").to(torch.float16)
    x = torch.randn((1, hidden), generator=g, device="cuda").to(torch.float16)
    y = torch.empty((1, hidden), dtype=torch.float16, device="cuda")
    ws = torch.zeros(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    per_expert = layers[0].experts.weight_bytes([0])
    step_bytes = 9 * per_expert  # 8 routed (distinct) + shared, all the same size

    # every rotating layer runs at least once before the timed loop (its first call builds its
    # expert pointer tables on the device)
    for i in range(max(args.warmup, L)):
        layers[i % L](x, scores[i % nrows], y=y, ws=ws)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record()
    for i in range(args.warmup, nsteps):
        layers[i % L](x, scores[i], y=y, ws=ws)
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    moe.check_status(ws)  # raises if a bounded in-kernel wait gave up during the timed steps

    # the same steps replayed from a HIP graph (one graph holds one step of each rotating layer):
    # removes host launch overhead, which is the production setting for decode
    stream = torch.cuda.Stream()
    ys = [torch.empty((1, hidden), dtype=torch.float16, device="cuda") for _ in range(L)]
    graph = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(graph, stream=stream):
        for li in range(L):
            layers[li](x, scores[li], y=ys[li], ws=ws)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(1, args.steps // L)
    g0, g1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    g0.record()
    for _ in range(reps):
        graph.replay()
    g1.record()
    torch.cuda.synchronize()
    ms_graph = g0.elapsed_time(g1) / (reps * L)
    moe.check_status(ws)

    # phase split with HIP events recorded inside the library on the layer's stream
    import ctypes as C
    lib.hx_profile_enable(1)
    for i in range(args.warmup, nsteps):
        layers[i % L](x, scores[i], y=y, ws=ws)
    tot = (C.c_double * 16)()
    cnt = (C.c_int * 16)()
    n = lib.hx_profile_read(tot, cnt, 16)
    lib.hx_profile_enable(0)
    phases = {}
    for p in range(n):
        if cnt[p]:
            phases[lib.hx_profile_phase_name(p).decode()] = tot[p] / cnt[p] * 1e3  # us per call
    # one persistent launch per layer (router, permutation, gate/up, SiLU-gate, down, ordered
    # reduction, shared combine): its bytes are the whole step's compressed weights
    dominant = ("moe_decode", step_bytes)
    dom_us = phases[dominant[0]]
    achieved = dominant[1] / (dom_us * 1e-6) / 1e9
    return {
        "ms_per_step": ms_graph, "value": step_bytes / (ms_graph * 1e-3) / 1e9, "step_bytes": step_bytes,
        "wall_s": wall, "ms_eager": ms, "graph_steps": reps * L,
        "phases_us": phases, "dominant": dominant[0], "dominant_bytes": dominant[1], "dominant_us": dom_us,
        "roofline_achieved": achieved, "layers": layers,
    }


def bench_prefill(args, torch, moe):
    E, hidden, inter, topk, T = 288, 4096, 2048, 8, 4096
    bits = [2 if e < E // 2 else 3 for e in range(E)]
    ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=77)
    layer = moe.MoeLayer(ex, None, topk=topk)
    scores = torch.from_numpy(zipf_scores(T, E, 1.1, seed=11)).cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(3)
    x = torch.randn((T, hidden), generator=g, device="cuda").to(torch.float16)
    y = torch.empty((T, hidden), dtype=torch.float16, device="cuda")
    ws = torch.zeros(layer.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    for _ in range(2):
        layer(x, scores, y=y, ws=ws)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = args.prefill_steps
    t0.record()
    for _ in range(reps):
        layer(x, scores, y=y, ws=ws)
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    flops = 2.0 * T * topk * 3 * hidden * inter
    del ws, layer, ex
    # the same workload with MCG-codebook experts (the reference's other MoE codebook)
    ex = moe.ExpertSet.synthetic(E, hidden, inter, bits, seed=78, mul1=False)
    layer = moe.MoeLayer(ex, None, topk=topk, mcg=True)
    ws = torch.zeros(layer.workspace_bytes(T), dtype=torch.uint8, device="cuda")
    for _ in range(2):
        layer(x, scores, y=y, ws=ws)
    torch.cuda.synchronize()
    t0.record()
    for _ in range(reps):
        layer(x, scores, y=y, ws=ws)
    t1.record()
    torch.cuda.synchronize()
    ms_mcg = t0.elapsed_time(t1) / reps
    del ws, layer, ex
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "flops": flops, "mcg_ms": ms_mcg}


def graph_time_us(torch, fn, reps: int = 20, inner: int = 20) -> float:
    """Average microseconds of one fn() call: `inner` calls captured back to back in one HIP graph,
    replayed `reps` times (one call per graph would add the replay's own launch cost, tens of us, to
    every µs-scale kernel).  fn must be capture-safe."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        fn()  # warm up on the capturing stream: its workspace is allocated outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(inner):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        graph.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (reps * inner) * 1e3


def bench_linears(torch, moe, exl3, only: str = ""):
    """BASELINE configs 1, 2 and 5a: single EXL3 linears (weight GB/s at M <= 16, TFLOP/s on MFMA)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    out = {}
    cases = [("config1_K4096_N2048_2bit_M1", 4096, 2048, 2, 1),
             ("config2_K4096_N12288_4bit_M1", 4096, 12288, 4, 1),
             ("config2_K4096_N12288_4bit_M4", 4096, 12288, 4, 4),
             ("config2_K4096_N12288_4bit_M8", 4096, 12288, 4, 8),
             ("config5a_lmhead_K4096_N151552_5bit_M1", 4096, 151552, 5, 1),
             ("config5a_lmhead_K4096_N151552_5bit_M512", 4096, 151552, 5, 512),
             # not a BASELINE config: a long dense 2-bit stream through the same decode core, the
             # steady-state decode rate that bounds the MoE decode layer's streaming phases
             ("stream_K16384_N32768_2bit_M1", 16384, 32768, 2, 1)]
    for name, K, N, bits, M in cases:
        if only not in name:
            continue
        copies = 4 if K * N * bits // 8 < 256 << 20 else 1   # rotate copies so the 256 MB MALL does not hold them
        ws_ = [exl3.GroupWords(*moe.synthetic_linear(K, N, bits, g), exl3.MUL1) for _ in range(copies)]
        x = torch.randn((M, K), generator=g, device="cuda").half()
        y = torch.empty((M, N), dtype=torch.float32, device="cuda")
        a_had = torch.empty((M, K), dtype=torch.float16, device="cuda") if M > exl3.GEMV_MAX_M else None

        def run():
            for w in ws_:
                exl3.gemm(y, x, w, M, N, K, bits, True, a_had=a_had)
        us = graph_time_us(torch, run) / copies
        wbytes = K * N * bits / 8 + 2 * K + 2 * N
        out[name] = {"us": round(us, 2), "weight_gbs": round(wbytes / us / 1e3, 1),
                     "pct_hbm": round(100 * wbytes / us / 1e3 / HBM_PEAK_GBS, 2),
                     "tflops": round(2.0 * M * K * N / us / 1e6, 2),
                     "tera_weights_per_s": round(K * N / us / 1e6, 2)}
        del ws_
    return out


def bench_sweep(torch, moe, layers_n: int = 42):
    """BASELINE config 5b: 42 resident MoE layers (288 routed x 2-bit experts + one 2-bit shared
    expert each), 1 token, independent seeded routing per layer; one step = the 42 layers back to
    back.  Bytes per layer: the 8 routed and the shared expert's compressed weights."""
    E, hidden, inter = 288, 4096, 2048
    layers = [moe.MoeLayer(moe.ExpertSet.synthetic(E, hidden, inter, 2, seed=20000 + i),
                           moe.synthetic_dense_mlp(hidden, inter, 2, seed=30000 + i), topk=8)
              for i in range(layers_n)]
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    scores = torch.randn((layers_n, 1, E), generator=g, device="cuda").half()
    x = torch.randn((1, hidden), generator=g, device="cuda").half()
    ys = [torch.empty((1, hidden), dtype=torch.float16, device="cuda") for _ in range(layers_n)]
    ws = torch.zeros(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")

    def run():
        for i in range(layers_n):
            layers[i](x, scores[i], y=ys[i], ws=ws)
    us = graph_time_us(torch, run, reps=10, inner=2)
    moe.check_status(ws)
    step_bytes = layers_n * 9 * layers[0].experts.weight_bytes([0])
    assert step_bytes == layers_n * 56954880
    del layers
    return {"layers": layers_n, "us_per_step": round(us, 1), "us_per_layer": round(us / layers_n, 2),
            "weight_gbs": round(step_bytes / us / 1e3, 1),
            "pct_hbm": round(100 * step_bytes / us / 1e3 / HBM_PEAK_GBS, 2), "bytes_per_step": step_bytes,
            "note": "8 routed + 1 shared expert per layer (42 x 56,954,880 B); weights of all 42 layers "
                    "resident (~72 GiB)"}


def cpu_baseline(layers, budget_s: float):
    """The C oracle's fp32 decode + GEMV (OpenMP over column tiles) over the same experts of the
    decode layer (gate, up, down of 8 routed + shared), timed on this host."""
    from oracle import oracle as O
    import torch
    lay = layers[0]
    ex, sh = lay.experts, lay.shared
    rng = np.random.default_rng(0)
    experts = [int(e) for e in rng.permutation(ex.num_experts)[:8]]
    mats = []
    for e in experts:
        for p, (K, N) in enumerate([(ex.hidden, ex.inter), (ex.hidden, ex.inter), (ex.inter, ex.hidden)]):
            mats.append((K, N, ex.bits[p][e], ex.trellis[p][e], ex.suh[p][e], ex.svh[p][e]))
    for p, w in enumerate(sh):
        K, N = w.in_features, w.out_features
        mats.append((K, N, w.bits, w.trellis, w.suh, w.svh))
    host = [(K, N, b, t.cpu().view(torch.int16).numpy().view(np.uint16), s.cpu().numpy(), v.cpu().numpy())
            for K, N, b, t, s, v in mats]
    x = {K: rng.standard_normal((1, K)).astype(np.float16) for K in {m[0] for m in host}}
    def run(threads, budget):
        total_s, total_bytes, layers_done = 0.0, 0, 0
        while total_s < budget and layers_done < 2000:
            for K, N, b, t, s, v in host:
                _, secs = O.cpu_linear_f32(x[K], t, s, v, K, N, b, 2, threads)
                total_s += secs
                total_bytes += t.size * 2 + s.size * 2 + v.size * 2
            layers_done += 1
        return total_bytes / total_s / 1e9, layers_done, total_s

    threads = O.cpu_max_threads()
    gbs, layers_done, total_s = run(threads, budget_s)
    gbs1, layers1, total1 = run(1, budget_s / 3)
    return {"value": gbs, "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"{layers_done} MoE decode layers (8 routed + shared experts, gate/up/down, 2-bit, 1 token) "
                      f"through oracle/exl3_oracle.c hx_cpu_linear_f32 (fp32 accumulate, OpenMP over {threads} "
                      f"threads), {total_s:.1f} s",
            "nproc": os.cpu_count(),
            "single_thread": {"value": gbs1, "unit": "GB/s", "cores": 1,
                              "sample": f"{layers1} layers of the same workload on one thread, {total1:.1f} s"}}


def traffic_from_profile(phase: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/moe_decode_layer_traffic.json, made by the command recorded in
    it), or None when that summary is absent."""
    from pathlib import Path
    f = Path(__file__).resolve().parent / "profiles" / "moe_decode_layer_traffic.json"
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return d["kernels"][phase]["hbm_bytes_per_launch"]
    except Exception:
        return None


def profile_only(torch, moe):
    """Workload for rocprofv3 --pmc runs: 3 plain copies of 256 MiB (the calibration kernel whose
    byte count is known), then 10 eager steps of the decode layer over 2 rotating layers."""
    src = torch.ones(64 << 20, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    # weights: device copies of host-generated random blocks (the counter-collection pass of
    # rocprofv3 is kept away from device RNG kernels)
    from helios_glm53flash_amd import exl3
    E, hidden, inter, bits = 288, 4096, 2048, 2
    r = np.random.default_rng(0)
    blk = torch.from_numpy(r.integers(-32768, 32768, size=hidden * inter // 8, dtype=np.int16)).cuda()
    sgn = torch.from_numpy(r.choice([-1.0, 1.0], 4096).astype(np.float16)).cuda()
    scl = torch.from_numpy((r.choice([-1.0, 1.0], 4096) * r.uniform(0.5, 1.5, 4096)).astype(np.float16)).cuda()

    def lin(K, N, off):
        t = torch.roll(blk, off).view(K // 16, N // 16, 16 * bits).clone()
        return t, sgn[:K].clone(), scl[:N].clone()

    shapes = [(hidden, inter), (hidden, inter), (inter, hidden)]
    layers = []
    for li in range(2):
        tr, su, sv, bt = [[], [], []], [[], [], []], [[], [], []], [[], [], []]
        for e in range(E):
            for p, (K, N) in enumerate(shapes):
                a, b_, c = lin(K, N, 8 * (li * 1000 + 3 * e + p))
                tr[p].append(a)
                su[p].append(b_)
                sv[p].append(c)
                bt[p].append(bits)
        sh = [exl3.GroupWords(*lin(K, N, 17 + p), exl3.MUL1) for p, (K, N) in enumerate(shapes)]
        layers.append(moe.MoeLayer(moe.ExpertSet(hidden, inter, tr, su, sv, bt, True), sh, topk=8))
    scores = torch.from_numpy(r.standard_normal((10, 1, E)).astype(np.float16)).cuda()
    x = torch.from_numpy(r.standard_normal((1, hidden)).astype(np.float16)).cuda()
    ws = torch.zeros(layers[0].workspace_bytes(1), dtype=torch.uint8, device="cuda")
    for i in range(10):
        layers[i % 2](x, scores[i], ws=ws)
    torch.cuda.synchronize()
    print("profile workload done: copy 256 MiB x3, 10 decode-layer steps")


def bench_router(torch):
    """Router logits (gemm_nt_f16, glue2.cu:9-65): fp16 scores [M][288] = x [M][4096] . W^T, W the
    router gate [288][4096] fp16 (2.36 MB); M = 1 (decode, HIP graph) and M = 4096 (prefill)."""
    from helios_glm53flash_amd import exl3
    E, H = 288, 4096
    r = np.random.default_rng(9)
    w = torch.from_numpy((r.standard_normal((E, H)) * 0.02).astype(np.float16)).cuda()
    out = {}
    for M in (1, 4096):
        x = torch.from_numpy(r.standard_normal((M, H)).astype(np.float16)).cuda()
        y = torch.empty((M, E), dtype=torch.float16, device="cuda")
        us = graph_time_us(torch, lambda: exl3.gemm_nt_f16(y, x, w, M, E, H))
        flops = 2.0 * M * E * H
        out[f"M{M}"] = {"us": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                        "weight_gbs": round(E * H * 2 / (us * 1e-6) / 1e9, 1)}
    return out


def bench_checkpoint(torch):
    """Checkpoint load rate: one config-3 layer (288 routed experts, 2-bit, 1.82 GB) written as two
    safetensors shards to a temporary directory, then validated and loaded into one HBM slab
    (helios_glm53flash_amd.checkpoint).  The file was just written, so it sits in the page cache:
    the rate is host memory -> pinned staging -> HBM plus validation, not disk."""
    import tempfile
    import time

    from safetensors.numpy import save_file

    from helios_glm53flash_amd import checkpoint as ck
    E, hidden, inter, bits = 288, 4096, 2048, 2
    r = np.random.default_rng(5)
    blk = r.integers(-32768, 32768, size=hidden * inter * bits // 16 + 4096, dtype=np.int16)
    sgn = r.choice([-1.0, 1.0], hidden).astype(np.float16)
    mul = np.array(0x83DCD12D - (1 << 32), dtype=np.int32)
    with tempfile.TemporaryDirectory() as d:
        for part in range(2):
            tensors = {}
            for e in range(part * E // 2, (part + 1) * E // 2):
                for p, (pn, (K, N)) in enumerate(zip(ck.PROJ_NAMES, ((hidden, inter), (hidden, inter),
                                                                      (inter, hidden)))):
                    base = f"model.language_model.layers.0.mlp.experts.{e}.{pn}"
                    o = (e * 3 + p) % 4096
                    tensors[base + ".trellis"] = blk[o:o + K * N * bits // 16].reshape(K // 16, N // 16, 16 * bits)
                    tensors[base + ".suh"] = sgn[:K]
                    tensors[base + ".svh"] = sgn[:N]
                    tensors[base + ".mul1"] = mul
            save_file(tensors, f"{d}/model-{part:05d}-of-00002.safetensors")
            del tensors
        t0 = time.perf_counter()
        ss = ck.ShardSet(d)
        ex = ck.load_experts(ss, 0, E, hidden, inter)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        nbytes = sum(t.numel() * t.element_size() for p in range(3) for arr in (ex.trellis[p], ex.suh[p], ex.svh[p])
                     for t in arr)
        del ex
    return {"workload": "checkpoint load: 288 experts x (gate, up, down) 2-bit, 2 shards, page-cache resident",
            "bytes": nbytes, "seconds": round(dt, 3), "gbs": round(nbytes / dt / 1e9, 2)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--layers", type=int, default=8, help="independent layers rotated over (MALL defeat)")
    ap.add_argument("--prefill-steps", type=int, default=5)
    ap.add_argument("--skip-prefill", action="store_true")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--skip-extra", action="store_true", help="skip the linear and 42-layer sweep configs")
    ap.add_argument("--profile-only", action="store_true",
                    help="counter-collection driver: a 256 MiB device copy (calibration), then eager decode steps")
    ap.add_argument("--linears-only", default=None, metavar="SUBSTR",
                    help="run only the linear cases whose name contains SUBSTR and print their results")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (one GPU holds every expert); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from helios_glm53flash_amd import moe
    from helios_glm53flash_amd._lib import lib

    torch.cuda.set_device(0)
    if args.profile_only:
        profile_only(torch, moe)
        return
    from helios_glm53flash_amd import exl3
    if args.linears_only is not None:
        print(json.dumps(bench_linears(torch, moe, exl3, args.linears_only)))
        return
    dec = bench_decode(args, torch, moe, lib)
    pre = None if args.skip_prefill else bench_prefill(args, torch, moe)
    lin = None if args.skip_extra else bench_linears(torch, moe, exl3)
    sweep = None if args.skip_extra else bench_sweep(torch, moe)
    ckpt = None if args.skip_extra else bench_checkpoint(torch)
    router = None if args.skip_extra else bench_router(torch)
    cpu = None if args.skip_cpu else cpu_baseline(dec["layers"], args.cpu_budget)

    out = {
        "metric": METRIC,
        "value": round(dec["value"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded uniform trellis words, +-1 suh, +-U(0.5,1.5) svh, N(0,1) activations and "
                "router logits; random-init weights of the GLM-5.3-Flash MoE layer shape)",
        "config": {
            "workload": "moe_decode_layer: 288 routed experts + 1 shared, hidden 4096, intermediate 2048, "
                        "2-bit EXL3 (mul1 codebook), sigmoid top-8 (scale 2.5), 1 token (BASELINE config 3)",
            "tokens": 1, "experts": 288, "topk": 8, "bits": 2, "hidden": 4096, "intermediate": 2048,
            "rotating_layers": args.layers, "bytes_per_step": dec["step_bytes"],
            "pct_of_hbm_peak": round(100.0 * dec["value"] / HBM_PEAK_GBS, 2),
        },
        "roofline": {
            "bound": "hbm",
            "traffic": traffic_from_profile(dec["dominant"]),
            "kernel": dec["dominant"],
            "achieved": round(dec["roofline_achieved"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dec["roofline_achieved"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": dec["dominant_bytes"],
            "avg_launch_us": round(dec["dominant_us"], 3),
        },
        "cpu_baseline": cpu,
        "extra": {
            "decode_phases_us": {k: round(v, 3) for k, v in dec["phases_us"].items()},
            "decode_eager_ms_per_step": round(dec["ms_eager"], 5),
            "decode_eager_gbs": round(dec["step_bytes"] / (dec["ms_eager"] * 1e-3) / 1e9, 2),
            "decode_timing": "value/ms_per_step: HIP-graph replay of the layer steps (%d steps); eager: one "
                             "host call per step" % dec["graph_steps"],
            "linears": lin,
            "sweep_42_layers": sweep,
            "checkpoint_load": ckpt,
            "router_logits": router,
            "prefill": None if pre is None else {
                "workload": "moe_prefill: 4096 tokens, top-8 of 288 with Zipf(1.1) popularity, experts 0-143 "
                            "2-bit / 144-287 3-bit, hidden 4096, intermediate 2048 (BASELINE config 4), routed "
                            "experts only",
                "ms": round(pre["ms"], 4), "tflops": round(pre["tflops"], 2),
                "pct_of_fp16_peak": round(100.0 * pre["tflops"] / FP16_PEAK_TFLOPS, 2),
                "roofline": {"bound": "mfma", "achieved": round(pre["tflops"], 2), "peak": FP16_PEAK_TFLOPS,
                             "unit": "TFLOP/s", "frac": round(pre["tflops"] / FP16_PEAK_TFLOPS, 4),
                             "flops_per_step": pre["flops"],
                             "note": "algorithmic 2*rows*K*N over the routed rows' gate, up and down GEMMs, "
                                     "per layer call (router, permutation, gather and combine included in "
                                     "the time)"},
                "mcg_ms": round(pre["mcg_ms"], 4),
                "mcg_note": "the same workload with MCG-codebook experts (mul1 is the headline codebook)",
            },
        },
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
