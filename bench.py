"""Benchmark of the nearest-neighbour hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-secondary] [--no-cpu]

Headline: one step = Chamfer forward + backward
(ChamferDistance('mean') and its gradient) at B=32, N=M=8192, float32, inputs
resident in HBM.  value = directed pair-distances per second (2*B*N*M per
step) in G/s.  The roofline object covers the dominant kernels, the Chamfer
forward as the module runs it (grid sort + exact grid search + the fused
mean's two small reduction kernels, timed together with HIP events on the
stream they run on, right after the timed steps): 9 FLOP per directed pair
of the brute-force algorithm against the 157.3 TFLOP/s FP32 peak, next to
the pairs the search actually evaluated; its traffic comes from the
FETCH_SIZE/WRITE_SIZE runs summarised in profiles/.  The CPU baseline is the reference's CPU formulation of Chamfer
(tests/test_chamfer.py:11-25 of the reference: broadcast, square, sum, min,
plus autograd backward), chunked, on a bounded sample, on the host's cores.

Secondary lines (other BASELINE configs, reported under "secondary"):
Chamfer c2 in float16, knn_points c3, knn_points c5 (bfloat16, matrix
cores), FPS c4 (ms), gather_points c4 fwd/bwd (GB/s), earth mover's
distance at B=16, N=M=2048 (ms, against the reference's published RTX 3090
time); the KNN, FPS and EMD lines carry a bounded CPU baseline of the
oracle's restatement of the reference kernels (oracle/).

Prints exactly one JSON line.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "torch-point-ops_amd"))
sys.path.insert(0, REPO)

FP32_PEAK_TFLOPS = 157.3
EMD_REF_MS = 32.366  # README.md:314, EMD FP32 eager, B16_N2048_M2048, RTX 3090
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0  # dense MFMA
FLOP_PER_PAIR = 9  # 3 sub + 3 mul + 2 add + 1 compare per directed pair


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def host_cores():
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# --------------------------------------------------------------------- GPU

def time_steps(fn, steps, warmup, torch):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def bench_chamfer(tpo, torch, steps, warmup):
    import workloads

    p1, p2 = workloads.chamfer_c2()
    B, N, _ = p1.shape
    M = p2.shape[1]
    dev = torch.device("cuda:0")
    a = p1.to(dev).requires_grad_(True)
    b = p2.to(dev).requires_grad_(True)

    model = tpo.ChamferDistance("mean")

    def step():
        # ChamferDistance('mean') forward + backward through autograd
        loss = model(a, b)
        return torch.autograd.grad(loss, (a, b))

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    sec = (time.perf_counter() - t0) / steps
    # the module's forward alone (sort, search and the loss kernels), HIP
    # events on the current stream, which is the one the op launches on
    # (events inside every step would add their own gaps to the step time)
    a0, b0 = a.detach(), b.detach()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        model(a0, b0)
    e1.record()
    torch.cuda.synchronize()
    out = dict(pairs=2 * B * N * M, sec=sec, B=B, N=N, M=M,
               loss_fwd_sec=e0.elapsed_time(e1) / steps / 1e3)
    out.update(chamfer_forward_paths(torch, a0, b0, steps))
    return out


def chamfer_forward_paths(torch, p1, p2, reps):
    """The forward alone through the C ABI, HIP events on the stream it runs
    on: with a workspace (exact grid search: sort + search launches) and
    without (dense filter kernel), plus the pairs the grid search evaluated."""
    import ctypes

    from torch_point_ops import _native

    lib = ctypes.CDLL(_native.HIP_LIB)
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.tpo_chamfer_fwd.argtypes = [ctypes.c_int, P, P, I, I, I, P, P, P, P, P, I, P]
    lib.tpo_chamfer_workspace_size.argtypes = [ctypes.c_int, I, I, I]
    lib.tpo_chamfer_workspace_size.restype = I
    lib.tpo_chamfer_pairs_evaluated.argtypes = [ctypes.c_int, P, I, I, I, P, P]
    B, N, M = p1.shape[0], p1.shape[1], p2.shape[1]
    dev = p1.device
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    d1, d2 = torch.empty(B, N, device=dev), torch.empty(B, M, device=dev)
    i1 = torch.empty(B, N, dtype=torch.int32, device=dev)
    i2 = torch.empty(B, M, dtype=torch.int32, device=dev)
    ws = torch.empty(lib.tpo_chamfer_workspace_size(0, B, N, M), dtype=torch.uint8, device=dev)

    def run(w):
        rc = lib.tpo_chamfer_fwd(0, p1.data_ptr(), p2.data_ptr(), B, N, M, d1.data_ptr(),
                                 d2.data_ptr(), i1.data_ptr(), i2.data_ptr(),
                                 None if w is None else w.data_ptr(),
                                 0 if w is None else w.numel(), sp)
        assert rc == 0

    res = {}
    for name, w in (("grid", ws), ("dense", None)):
        for _ in range(3):
            run(w)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            run(w)
        e1.record(stream)
        torch.cuda.synchronize()
        res[name + "_fwd_sec"] = e0.elapsed_time(e1) / reps / 1e3
    run(ws)
    pairs = torch.zeros(1, dtype=torch.int64, device=dev)
    assert lib.tpo_chamfer_pairs_evaluated(0, ws.data_ptr(), B, N, M, pairs.data_ptr(), sp) == 0
    torch.cuda.synchronize()
    res["pairs_evaluated"] = int(pairs.item())
    return res


def bench_chamfer_fp16(tpo, torch, steps):
    """Config 2's float16 variant: ChamferDistance('mean') forward + backward."""
    import workloads

    p1, p2 = workloads.chamfer_c2(dtype=torch.float16)
    dev = torch.device("cuda:0")
    a = p1.to(dev).requires_grad_(True)
    b = p2.to(dev).requires_grad_(True)
    model = tpo.ChamferDistance("mean")
    sec = time_steps(lambda: torch.autograd.grad(model(a, b), (a, b)), steps, 2, torch)
    return dict(pairs=2 * a.shape[0] * a.shape[1] * b.shape[1], sec=sec)


def bench_knn(tpo, torch, steps):
    import workloads

    p1, p2, l1, l2 = workloads.knn_c3()
    dev = torch.device("cuda:0")
    a, b, la, lb = p1.to(dev), p2.to(dev), l1.to(dev), l2.to(dev)
    mod = tpo.KNearestNeighbors(K=16, return_nn=True)
    raw = lambda: torch.ops.torch_point_ops_knn.knn_forward(a, b, la, lb, 2, 16, -1)  # noqa
    sec_mod = time_steps(lambda: mod(a, b, la, lb), steps, 2, torch)
    sec_raw = time_steps(raw, steps, 2, torch)
    pairs = int((l1 * l2).sum())
    return dict(pairs=pairs, sec_module=sec_mod, sec_kernel=sec_raw)


def bench_knn_c5(tpo, torch, steps):
    """Config 5: high-D KNN, bfloat16 inputs on the matrix cores; also one run
    of the reference-semantics float kernel (version 0) on the widened inputs."""
    import workloads

    q, r = workloads.knn_c5()
    dev = torch.device("cuda:0")
    a, b = q.to(dev), r.to(dev)
    B, P1, D = a.shape
    P2 = b.shape[1]
    la = torch.full((B,), P1, dtype=torch.int64, device=dev)
    lb = torch.full((B,), P2, dtype=torch.int64, device=dev)
    op = torch.ops.torch_point_ops_knn.knn_forward
    sec = time_steps(lambda: op(a, b, la, lb, 2, 32, -1), steps, 2, torch)
    af, bf = a.float(), b.float()
    sec_f32 = time_steps(lambda: op(af, bf, la, lb, 2, 32, -1), 1, 1, torch)
    return dict(pairs=B * P1 * P2, D=D, sec=sec, sec_f32=sec_f32)


def bench_fps(tpo, torch, steps):
    import workloads

    pts = workloads.fps_c4().to("cuda:0")
    sec = time_steps(lambda: tpo.furthest_point_sampling(pts, 4096), steps, 2, torch)
    idx = tpo.furthest_point_sampling(pts, 4096)
    feats, go = workloads.gather_c4()
    f = feats.to("cuda:0")
    g = go.to("cuda:0")
    fwd = time_steps(lambda: torch.ops.torch_point_ops_fps.gather_points_forward(f, idx),
                     steps * 10, 3, torch)
    bwd = time_steps(lambda: torch.ops.torch_point_ops_fps.gather_points_backward(g, idx, 65536),
                     steps * 10, 3, torch)
    B, N, m = pts.shape[0], pts.shape[1], 4096
    C, M = f.shape[1], 4096
    return dict(fps_sec=sec, updates=B * N * (m - 1), gather_fwd_sec=fwd, gather_bwd_sec=bwd,
                fwd_bytes=B * M * 8 + 2 * B * C * M * 4,
                bwd_bytes=B * C * N * 4 + B * C * M * 4 + B * M * 8, idx=idx.cpu(), pts=pts.cpu())


def bench_emd(tpo, torch, steps):
    """earth_movers_distance forward (no grad, as benchmark_flops.py:146-160
    times it) and EarthMoverDistance forward + backward at B=16, N=M=2048."""
    import workloads

    a, b = (t.to("cuda:0") for t in workloads.emd_b16())

    def fwd():
        with torch.no_grad():
            tpo.earth_movers_distance(a, b)

    sec = time_steps(fwd, steps, 3, torch)
    ga = a.clone().requires_grad_(True)
    gb = b.clone().requires_grad_(True)
    mod = tpo.EarthMoverDistance()
    sec_fb = time_steps(lambda: torch.autograd.grad(mod(ga, gb), (ga, gb)), steps, 2, torch)
    return dict(sec=sec, sec_fb=sec_fb, B=a.shape[0], N=a.shape[1], M=b.shape[1])


# --------------------------------------------------------------------- CPU

def cpu_chamfer(torch, budget_s=12.0):
    """Reference CPU formulation (test_chamfer.py:11-25) + autograd backward,
    query-chunked, on whole clouds of config 2 until the budget is used."""
    import workloads

    p1, p2 = workloads.chamfer_c2()
    threads = torch.get_num_threads()

    def one_cloud(b):
        a = p1[b:b + 1].clone().requires_grad_(True)
        c = p2[b:b + 1].clone().requires_grad_(True)
        mins1, mins2 = [], None
        for s in range(0, a.shape[1], 512):
            dm = ((a[:, s:s + 512].unsqueeze(2) - c.unsqueeze(1)) ** 2).sum(3)
            mins1.append(dm.min(2).values)
            m2 = dm.min(1).values
            mins2 = m2 if mins2 is None else torch.minimum(mins2, m2)
        d1 = torch.cat(mins1, 1)
        loss = d1.mean() + mins2.mean()
        loss.backward()

    t0 = time.perf_counter()
    n = 0
    while True:
        one_cloud(n % p1.shape[0])
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= p1.shape[0]:
            break
    sec = time.perf_counter() - t0
    pairs = 2 * n * p1.shape[1] * p2.shape[1]
    return dict(value=pairs / sec / 1e9, unit="G pair-dists/s", cores=threads, kind="port",
                sample=f"{n} of 32 clouds of config 2 (8192x8192 each, both directions, "
                       f"fwd+bwd) with the reference tests' torch formulation, "
                       f"512-query chunks, {threads} torch threads on {cpu_model()}")


def cpu_knn(O, np, threads):
    import workloads

    p1, p2, l1, l2 = workloads.knn_c3()
    q = 64  # queries per cloud
    a = p1[:, :q].numpy()
    ln1 = np.minimum(l1.numpy(), q)
    t0 = time.perf_counter()
    O.cpu_knn_fwd(a, p2.numpy(), ln1, l2.numpy(), 16, 2, nthreads=threads)
    sec = time.perf_counter() - t0
    pairs = float((ln1 * l2.numpy()).sum())
    return dict(value=pairs / sec / 1e9, unit="G pair-dists/s", cores=threads, kind="port",
                sample=f"{q} queries per cloud x 8 clouds of config 3 (knn.cpp restated)")


def cpu_knn_c5(O, np, threads):
    import workloads

    q, r = workloads.knn_c5()
    nq = 16  # queries per cloud
    a = q[:, :nq].float().numpy()
    b = r.float().numpy()
    ln1 = np.full(a.shape[0], nq, dtype=np.int64)
    ln2 = np.full(a.shape[0], b.shape[1], dtype=np.int64)
    t0 = time.perf_counter()
    O.cpu_knn_fwd(a, b, ln1, ln2, 32, 2, nthreads=threads)
    sec = time.perf_counter() - t0
    pairs = float(a.shape[0] * nq * b.shape[1])
    return dict(value=pairs / sec / 1e9, unit="G pair-dists/s", cores=threads, kind="port",
                sample=f"{nq} queries per cloud x 4 clouds of config 5 widened to float "
                       f"(knn.cpp restated; the reference CPU path has no bfloat16)")


def cpu_fps(O, np, pts, threads):
    nc = min(threads, pts.shape[0])
    m = 512
    t0 = time.perf_counter()
    O.cpu_fps(pts[:nc].numpy(), m, nthreads=nc)
    sec = time.perf_counter() - t0
    upd = nc * pts.shape[1] * (m - 1)
    return dict(value=upd / sec / 1e9, unit="G point-updates/s", cores=nc, kind="port",
                sample=f"{nc} clouds of config 4, first {m} samples, one thread per cloud "
                       f"(fps.cpp restated)")


def cpu_emd(O, threads):
    """The oracle's restatement of emd.cu's approxmatch + matchcost (the
    reference has no CPU kernel), one cloud per thread."""
    import workloads

    a, b = workloads.emd_b16()
    nc = max(1, min(threads, a.shape[0]))
    t0 = time.perf_counter()
    O.emd_fwd(a[:nc].numpy(), b[:nc].numpy())
    sec = time.perf_counter() - t0
    return dict(value=round(nc / sec, 3), unit="clouds/s", cores=nc, kind="port",
                sample=f"{nc} of the 16 clouds (2048 x 2048, float32), one per OpenMP thread, "
                       f"oracle/tpo_oracle.c restating emd.cu:18-230")


# ---------------------------------------------------------------- profiling

def profile_run(tpo, torch, reps=5):
    """Fixed kernel sequence for rocprofv3 (--kernel-trace / --pmc runs):
    every hot kernel at its BASELINE shape, plus a plain streaming copy of
    256 MiB (read 256 MiB, write 256 MiB) that calibrates the byte counters."""
    import workloads

    dev = torch.device("cuda:0")
    p1, p2 = (t.to(dev).requires_grad_(True) for t in workloads.chamfer_c2())
    k1, k2, l1, l2 = (t.to(dev) for t in workloads.knn_c3())
    h1, h2 = (t.to(dev) for t in workloads.knn_c5())
    hl1 = torch.full((h1.shape[0],), h1.shape[1], dtype=torch.int64, device=dev)
    hl2 = torch.full((h1.shape[0],), h2.shape[1], dtype=torch.int64, device=dev)
    pts = workloads.fps_c4().to(dev)
    feats, go = (t.to(dev) for t in workloads.gather_c4())
    src = torch.randn(64 << 20, device=dev)  # 256 MiB of float32
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.autograd.grad(tpo.ChamferDistance("mean")(p1, p2), (p1, p2))
        torch.ops.torch_point_ops_knn.knn_forward(k1, k2, l1, l2, 2, 16, -1)
        torch.ops.torch_point_ops_knn.knn_forward(h1, h2, hl1, hl2, 2, 32, -1)
        idx = tpo.furthest_point_sampling(pts, 4096)
        torch.ops.torch_point_ops_fps.gather_points_forward(feats, idx)
        torch.ops.torch_point_ops_fps.gather_points_backward(go, idx, 65536)
        torch.add(src, 0.0, out=dst)  # calibration copy
    torch.cuda.synchronize()
    print("profile run done", flush=True)


def profile_emd(tpo, torch, reps=5):
    """EMD forward + backward at B=16, N=M=2048, float32, for rocprofv3."""
    import workloads

    a, b = (t.to("cuda:0").requires_grad_(True) for t in workloads.emd_b16())
    mod = tpo.EarthMoverDistance()
    for _ in range(reps):
        torch.autograd.grad(mod(a, b), (a, b))
    torch.cuda.synchronize()
    print("profile emd done", flush=True)


# -------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-run", action="store_true",
                    help="run the fixed kernel sequence for rocprofv3 and exit")
    ap.add_argument("--profile-emd", action="store_true",
                    help="run EMD forward + backward (B=16, N=M=2048) for rocprofv3 and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build runs on a single MI355X "
              "(the sharding design is described in DESIGN.md); use --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import torch_point_ops as tpo

    if args.profile_run:
        profile_run(tpo, torch)
        return
    if args.profile_emd:
        profile_emd(tpo, torch)
        return
    log("[bench] chamfer c2 fwd+bwd")
    ch = bench_chamfer(tpo, torch, args.steps, args.warmup)
    value = ch["pairs"] / ch["sec"] / 1e9
    achieved = FLOP_PER_PAIR * ch["pairs"] / ch["loss_fwd_sec"] / 1e12
    executed = FLOP_PER_PAIR * ch["pairs_evaluated"] / ch["loss_fwd_sec"] / 1e12
    dense = FLOP_PER_PAIR * ch["pairs"] / ch["dense_fwd_sec"] / 1e12
    traffic = None
    tfile = os.path.join(REPO, "profiles", "chamfer_grid_fwd_c2_traffic.json")
    if os.path.exists(tfile):
        traffic = json.load(open(tfile)).get("hbm_bytes_per_launch")

    out = {
        "metric": "Chamfer/KNN G pair-dists/s & % FP32 VALU peak; FPS ms at N=64K->4K",
        "value": round(value, 3),
        "unit": "G pair-dists/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ch["sec"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (BASELINE configs[1] generator, seed 2)",
        "config": {"workload": "chamfer_distance fwd+bwd, B=32, N=M=8192, D=3, fp32, "
                               "ChamferDistance('mean') (BASELINE.json configs[1])",
                   "global_batch": ch["B"], "points": [ch["N"], ch["M"]],
                   "pairs_per_step": ch["pairs"], "parallelism": "single GPU"},
        "roofline": {"bound": "mfma",
                     "compute_unit": "VALU (fp32 vector ALU; 157.3 TFLOP/s is MI355X's fp32 peak)",
                     "kernel": "chamfer_grid_sort_kernel<float,8> + chamfer_grid_search_kernel"
                               "<float,256> + chamfer_loss_part_kernel<float,true> (the "
                               "module's fused mean)",
                     "achieved": round(achieved, 3), "peak": FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_PEAK_TFLOPS, 4),
                     "traffic": traffic, "fwd_ms": round(ch["loss_fwd_sec"] * 1e3, 4),
                     "fwd_ms_storing_distances": round(ch["grid_fwd_sec"] * 1e3, 4),
                     "flop_per_pair": FLOP_PER_PAIR, "algorithmic_pairs": ch["pairs"],
                     "pairs_evaluated": ch["pairs_evaluated"],
                     "executed_tflops": round(executed, 4),
                     "executed_frac": round(executed / FP32_PEAK_TFLOPS, 5),
                     "note": "achieved = 9 FLOP x all 2BNM directed pairs / forward time; the "
                             "exact grid search evaluates only pairs_evaluated of them, so frac "
                             "> 1 means less work than brute force (executed_* is the VALU "
                             "use); the brute-force kernel's own roofline is "
                             "secondary.chamfer_dense_c2"},
    }
    threads = min(host_cores(), int(os.environ.get("OMP_NUM_THREADS", host_cores())))
    if not args.no_cpu:
        log("[bench] cpu baseline (chamfer)")
        torch.set_num_threads(threads)
        out["cpu_baseline"] = cpu_chamfer(torch)
    if not args.no_secondary:
        from oracle import oracle as O

        sec = {"chamfer_dense_c2": {
            "kernel": "chamfer_fwd_filter_kernel<8,16>", "fwd_ms": round(ch["dense_fwd_sec"] * 1e3, 4),
            "achieved_tflops": round(dense, 3), "frac_fp32_peak": round(dense / FP32_PEAK_TFLOPS, 4)}}
        log("[bench] chamfer c2 fp16")
        h = bench_chamfer_fp16(tpo, torch, max(3, args.steps // 4))
        sec["chamfer_c2_fp16"] = {"ms_per_step": round(h["sec"] * 1e3, 4),
                                  "G_pair_dists_per_s": round(h["pairs"] / h["sec"] / 1e9, 2),
                                  "note": "fwd+bwd of ChamferDistance('mean'), float16 inputs, "
                                          "half arithmetic (exact grid search with half "
                                          "rounding margins)"}
        log("[bench] knn c3")
        kn = bench_knn(tpo, torch, max(3, args.steps // 4))
        sec["knn_c3"] = {"G_pair_dists_per_s_kernel": round(kn["pairs"] / kn["sec_kernel"] / 1e9, 2),
                         "G_pair_dists_per_s_module": round(kn["pairs"] / kn["sec_module"] / 1e9, 2),
                         "ms_kernel": round(kn["sec_kernel"] * 1e3, 3),
                         "ms_module_return_nn": round(kn["sec_module"] * 1e3, 3),
                         "frac_fp32_peak": round(FLOP_PER_PAIR * kn["pairs"] / kn["sec_kernel"]
                                                 / 1e12 / FP32_PEAK_TFLOPS, 4)}
        log("[bench] knn c5 (bf16, matrix cores)")
        k5 = bench_knn_c5(tpo, torch, max(3, args.steps // 4))
        mfma = 2 * k5["D"] * k5["pairs"] / k5["sec"] / 1e12
        sec["knn_c5_bf16"] = {"ms": round(k5["sec"] * 1e3, 3),
                              "G_pair_dists_per_s": round(k5["pairs"] / k5["sec"] / 1e9, 2),
                              "mfma_tflops": round(mfma, 2),
                              "frac_bf16_dense_peak": round(mfma / BF16_PEAK_TFLOPS, 4),
                              "ms_float_reference_semantics": round(k5["sec_f32"] * 1e3, 3)}
        log("[bench] fps + gather c4")
        fp = bench_fps(tpo, torch, max(3, args.steps // 4))
        sec["fps_c4"] = {"ms": round(fp["fps_sec"] * 1e3, 3),
                         "G_point_updates_per_s": round(fp["updates"] / fp["fps_sec"] / 1e9, 2)}
        sec["gather_c4"] = {
            "fwd_us": round(fp["gather_fwd_sec"] * 1e6, 2),
            "fwd_GBs": round(fp["fwd_bytes"] / fp["gather_fwd_sec"] / 1e9, 1),
            "bwd_us": round(fp["gather_bwd_sec"] * 1e6, 2),
            "bwd_GBs": round(fp["bwd_bytes"] / fp["gather_bwd_sec"] / 1e9, 1),
            "bwd_frac_hbm": round(fp["bwd_bytes"] / fp["gather_bwd_sec"] / 1e9 / HBM_PEAK_GBS, 3)}
        log("[bench] emd b16 n2048")
        em = bench_emd(tpo, torch, max(3, args.steps // 4))
        sec["emd_b16_n2048"] = {
            "ms_fwd": round(em["sec"] * 1e3, 3),
            "ms_fwd_bwd": round(em["sec_fb"] * 1e3, 3),
            "clouds_per_s": round(em["B"] / em["sec"], 1),
            "reference_rtx3090_ms_fwd": EMD_REF_MS,
            "speedup_vs_reference_rtx3090": round(EMD_REF_MS / (em["sec"] * 1e3), 2),
            "note": "earth_movers_distance forward under no_grad (the reference benchmark's "
                    "timing, README.md:314 quotes 32.366 ms eager fp32 on an RTX 3090) and "
                    "EarthMoverDistance fwd+bwd; float32, torch.randn clouds"}
        if not args.no_cpu:
            log("[bench] cpu baselines (knn, fps, emd)")
            sec["emd_b16_n2048"]["cpu_baseline"] = cpu_emd(O, threads)
            sec["knn_c3"]["cpu_baseline"] = cpu_knn(O, np, threads)
            sec["fps_c4"]["cpu_baseline"] = cpu_fps(O, np, fp["pts"], threads)
            sec["knn_c5_bf16"]["cpu_baseline"] = cpu_knn_c5(O, np, threads)
        out["secondary"] = sec
    out["host"] = {"cpu": cpu_model(), "cores": threads,
                   "gpu": torch.cuda.get_device_name(0)}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
