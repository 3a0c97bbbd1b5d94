"""Headline benchmark: MLP-4096 training samples/s on one MI355X + GEMM fraction of fp32 MFMA peak.

Workload (benchmark configuration C4, "Wide MLP-4096"): 4096 -> 4096 x4 hidden -> 4096, fp32, ReLU,
MSE loss, SGD momentum 0.9, batch 4096; X, Y ~ N(0,1), He-normal init from a seed; 10 warmup and
100 timed steps by default. A step is one full training step of the device-resident program:
5 forward GEMMs with fused bias+ReLU, the MSE loss and gradient, 5 dW GEMMs, 4 dX GEMMs with the
ReLU gradient fused, 5 bias column sums, and the transactional single-pass SGD-momentum update of
all 83,906,560 parameters into the other half of the double-buffered parameter set. Inputs are resident in HBM before the timed region; each step is one
synchronous program run (device work complete on return).

Per-step device times come from HIP events recorded on the context stream around every program
step during the timed region; the roofline object reports the GEMM steps (14 x 137.44 GFLOP).
The CPU baseline runs the C oracle (a single-threaded restatement of the reference's default
scalar CPU route) on a bounded sample of the same network (see cpu_baseline.sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

WIDTH = 4096
BATCH = 4096
LAYERS = 5
LR = 0.01
MOMENTUM = 0.9
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
HBM_PEAK_GBS = 8000.0


def gemm_flops() -> float:
    return 2.0 * BATCH * WIDTH * WIDTH


def measured_gemm_traffic():
    """HBM bytes per 4096^3 GEMM launch from the committed rocprofv3 --pmc summary, or None."""
    f = ROOT / "profiles" / "gemm_f32_v2_4096_traffic.md"
    try:
        for line in f.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def build_session(ctx, seed=0):
    from synaptik_amd.training import HipTrainingSession, MlpSpec, Sgd, init_parameters
    spec = MlpSpec.chain([WIDTH] * (LAYERS + 1), hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, seed, "builder_he_normal")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(LR, momentum=MOMENTUM), BATCH)
    rng = np.random.default_rng(seed + 1)
    x = ctx.upload(rng.standard_normal((BATCH, WIDTH), dtype=np.float32))
    y = ctx.upload(rng.standard_normal((BATCH, WIDTH), dtype=np.float32))
    return spec, Ws, bs, sess, x, y


def cpu_baseline(sample_batch: int, seed=0) -> dict:
    """Times the oracle on `sample_batch` rows of the same network plus one full update."""
    from oracle import oracle
    from synaptik_amd.training import MlpSpec, init_parameters
    spec = MlpSpec.chain([WIDTH] * (LAYERS + 1), hidden="relu", loss="mse")
    Ws, bs = init_parameters(spec, seed, "builder_he_normal")
    model = oracle.OracleMLP(Ws, bs, ["relu"] * (LAYERS - 1) + [None], "mse",
                             dict(kind="sgd", lr=LR, momentum=MOMENTUM))
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((sample_batch, WIDTH), dtype=np.float32)
    y = rng.standard_normal((sample_batch, WIDTH), dtype=np.float32)
    t0 = time.perf_counter()
    loss, gW, gb, _ = model.gradients(x, y)
    t_fb = time.perf_counter() - t0
    params = model.W + model.b
    grads = gW + gb
    t0 = time.perf_counter()
    for i, (p, g) in enumerate(zip(params, grads)):
        oracle.sgd_stage(p, g, model.m[i], lr=LR, momentum=MOMENTUM, completed_steps=1)
    t_upd = time.perf_counter() - t0
    step_s = (BATCH / sample_batch) * t_fb + t_upd
    return {
        "value": BATCH / step_s,
        "unit": "samples/s",
        **host_cores(),
        "kind": "port",
        "extrapolated": True,
        "sample": (f"oracle forward+backward of MLP-4096 on {sample_batch} of the 4096 rows "
                   f"({t_fb:.2f} s, scaled x{BATCH / sample_batch:.2f}) + one full SGD-momentum stage "
                   f"of all parameters ({t_upd:.2f} s): {step_s:.1f} s per 4096-sample step"),
    }


def openblas_baseline(threads: int, sample_batch: int, seed=0) -> dict:
    """The reference's OpenBLAS route restated (OpenBlasGemmInvocation.java:41-68: sgemm on
    row-major operands, single-threaded as qualifiedSingleThread, CpuBackendComposition.java:546-550)
    with numpy's bundled OpenBLAS: the 14 GEMMs of an MLP-4096 step on `sample_batch` rows, scaled
    to 4096 rows, plus ReLU, the MSE gradient and the SGD-momentum update in numpy. Reported beside
    the reference's default (scalar) route; not the reference's own code."""
    from threadpoolctl import threadpool_info, threadpool_limits
    rng = np.random.default_rng(seed)
    W = [rng.standard_normal((WIDTH, WIDTH), dtype=np.float32) * np.float32(0.02) for _ in range(LAYERS)]
    b = [np.zeros(WIDTH, np.float32) for _ in range(LAYERS)]
    x = rng.standard_normal((sample_batch, WIDTH), dtype=np.float32)
    y = rng.standard_normal((sample_batch, WIDTH), dtype=np.float32)
    with threadpool_limits(limits=threads, user_api="blas"):
        _ = x @ W[0].T  # warm the BLAS thread pool and its buffers
        t0 = time.perf_counter()
        acts = [x]
        for i in range(LAYERS):
            z = acts[-1] @ W[i].T + b[i]
            acts.append(np.maximum(z, 0) if i < LAYERS - 1 else z)
        dz = (acts[-1] - y) * np.float32(2.0 / acts[-1].size)
        grads = []
        for i in reversed(range(LAYERS)):
            grads.append((dz.T @ acts[i], dz.sum(0)))
            if i > 0:
                dz = (dz @ W[i]) * (acts[i] > 0)
        t_fb = time.perf_counter() - t0
        t0 = time.perf_counter()
        for (gw, gb), w, bb in zip(grads, reversed(W), reversed(b)):
            for p, g in ((w, gw), (bb, gb)):
                m = g.copy()            # first step: the momentum slot takes the gradient
                p -= np.float32(LR) * m
        t_upd = time.perf_counter() - t0
    step_s = (BATCH / sample_batch) * t_fb + t_upd
    version = next((i.get("version") for i in threadpool_info() if i["internal_api"] == "openblas"), None)
    return {"value": BATCH / step_s, "unit": "samples/s", "threads": threads,
            "nproc": host_cores()["nproc"], "extrapolated": sample_batch < BATCH,
            "kind": "openblas route (numpy's OpenBLAS %s), not the reference's default route" % version,
            "sample": (f"{sample_batch} of the 4096 rows ({t_fb:.2f} s, scaled x{BATCH / sample_batch:.0f}) "
                       f"+ one full SGD update ({t_upd:.2f} s)")}


def probe() -> int:
    """Small fixed workload for rocprofv3 --pmc runs: FETCH_SIZE / WRITE_SIZE of the GEMM are
    scaled by the same counters read for a plain copy kernel of known size."""
    from synaptik_amd.native import HipContext, HipProgram
    from synaptik_amd.program import ProgramBuilder
    ctx = HipContext(0)
    rng = np.random.default_rng(0)
    pb = ProgramBuilder()
    a = pb.input(BATCH * WIDTH)
    w = pb.input(WIDTH * WIDTH)
    c = pb.output(BATCH * WIDTH)
    pb.gemm(a, w, c, BATCH, WIDTH, WIDTH, trans_b=True)
    gemm = HipProgram(ctx, pb.image())
    A = ctx.upload(rng.standard_normal(BATCH * WIDTH, dtype=np.float32))
    W = ctx.upload(rng.standard_normal(WIDTH * WIDTH, dtype=np.float32))
    C = ctx.buffer(BATCH * WIDTH * 4)
    n_copy = 64 * 1024 * 1024  # 256 MiB read + 256 MiB written
    pc = ProgramBuilder()
    src = pc.input(n_copy)
    dst = pc.output(n_copy)
    pc.copy(src, dst, n_copy)
    copy = HipProgram(ctx, pc.image())
    S = ctx.upload(np.ones(n_copy, np.float32))
    D = ctx.buffer(n_copy * 4)
    for _ in range(3):
        gemm.run([A, W], [C])
        copy.run([S], [D])
    print(json.dumps({"probe": "ok", "gemm_algorithmic_bytes": (2 * BATCH * WIDTH + WIDTH * WIDTH) * 4,
                      "copy_bytes_each_way": n_copy * 4}), flush=True)
    ctx.close()
    return 0


def c3_line(ctx, rng, one_stream: bool = False) -> dict:
    """C3: 784 -> 1024 -> 1024 -> 10 classifier, softmax-CE, Adam, batch 1024: the configuration's
    50-step run (objective after its first and last step; it also captures the step's graphs),
    then 200 more steps timed. one_stream: the program's steps on one stream (for kernel traces
    whose per-kernel times are not shared with concurrent work)."""
    from synaptik_amd.training import Adam, HipTrainingSession, MlpSpec, init_parameters
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 0, "builder_he_normal")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Adam(1e-3, 0.9, 0.999, 1e-8), 1024)
    if one_stream:
        sess.program.set_concurrent(False)
    xb = ctx.upload(rng.uniform(0, 1, (1024, 784)).astype(np.float32))
    yb = ctx.upload(rng.integers(0, 10, 1024).astype(np.int64))
    sess.run_resident(xb, yb)
    first = float(sess.objective())
    for _ in range(49):
        sess.run_resident(xb, yb)
    last = float(sess.objective())
    t0 = time.perf_counter()
    for _ in range(200):
        sess.run_resident(xb, yb)
    wall = time.perf_counter() - t0
    sess.close()
    return {"samples_per_s": round(200 * 1024 / wall, 1), "ms_per_step": round(wall / 200 * 1e3, 4),
            "objective_step1": first, "objective_step50": last, "timed": "steps 51-250",
            "streams": 1 if one_stream else 2}


def gemm_layouts(ctx, reps: int = 20, warmup: int = 10) -> dict:
    """Plain GEMMs (no epilogue work beyond the store) in the four operand layouts, per shape:
    TFLOP/s from HIP events around each launch. The four programs are warmed up and then run in
    rotation, so that a clock or thermal drift falls on every layout alike. The training step's
    dW launches are TN with a fused optimizer update; this isolates the layout itself."""
    from synaptik_amd.native import HipProgram
    from synaptik_amd.program import ProgramBuilder
    rng = np.random.default_rng(0)
    out = {}
    layouts = (("NT", (0, 1)), ("NN", (0, 0)), ("TN", (1, 0)), ("TT", (1, 1)))
    for (M, N, K) in ((4096, 4096, 4096), (8192, 1024, 1024), (1024, 1024, 1024)):
        A = ctx.upload(rng.standard_normal(M * K, dtype=np.float32))
        B = ctx.upload(rng.standard_normal(K * N, dtype=np.float32))
        C = ctx.buffer(M * N * 4)
        progs = {}
        for name, (ta, tb) in layouts:
            pb = ProgramBuilder()
            a, b, c = pb.input(M * K), pb.input(K * N), pb.output(M * N)
            pb.gemm(a, b, c, M, N, K, trans_a=bool(ta), trans_b=bool(tb))
            progs[name] = HipProgram(ctx, pb.image())
        for _ in range(warmup):
            for prog in progs.values():
                prog.run([A, B], [C])
        for prog in progs.values():
            prog.set_profiling(True)
        for _ in range(reps):
            for prog in progs.values():
                prog.run([A, B], [C])
        row = {}
        for name, prog in progs.items():
            t, runs = prog.step_times()
            row[name] = round(2 * M * N * K / (t[0] / runs * 1e-3) / 1e12, 2)
            prog.close()
        for x in (A, B, C):
            x.close()
        out[f"{M}x{N}x{K}"] = row
    return out


def secondary(ctx, reps: int = 5, cpu: bool = True) -> dict:
    """The other benchmark configurations, measured on the same context (not the headline value)."""
    from synaptik_amd.native import HipProgram
    from synaptik_amd.program import ProgramBuilder
    from synaptik_amd.training import (Adam, HipTrainingSession, MlpSpec, Sgd, init_parameters,
                                       lower_dense_layer)
    out = {}
    rng = np.random.default_rng(7)
    # The box's attainable HBM rate for one read and one write per element: the library's copy
    # (one float4 per thread, streamed) over 1 GiB. Softmax forward moves the same bytes per
    # element; it is reported against this figure and against the nominal 8 TB/s.
    n = 1 << 28
    pb = ProgramBuilder()
    ca, cb = pb.input(n), pb.output(n)
    pb.copy(ca, cb, n)
    prog = HipProgram(ctx, pb.image())
    ba, bb = ctx.buffer(n * 4), ctx.buffer(n * 4)
    prog.run([ba], [bb])
    prog.set_profiling(True)
    for _ in range(reps * 4):
        prog.run([ba], [bb])
    t, runs = prog.step_times()
    copy_ms = t[0] / runs
    copy_gbs = 2 * n * 4 / copy_ms / 1e6
    out["hbm_copy_ceiling"] = {"bytes": 2 * n * 4, "ms": round(copy_ms, 4),
                               "GBps": round(copy_gbs, 1),
                               "frac_hbm": round(copy_gbs / HBM_PEAK_GBS, 4)}
    prog.close()
    ba.close()
    bb.close()
    # C5: softmax + LSE + mean forward, softmax-with-LSE-cotangent backward over [65536, 4096]
    R, C = 65536, 4096
    pb = ProgramBuilder()
    sx, sdp = pb.input(R * C), pb.input(R * C)
    sp, sl, sm, sdx = pb.output(R * C), pb.output(R), pb.output(1), pb.output(R * C)
    pb.softmax(sx, sp, R, C, lse=sl)
    pb.reduce_all(sl, sm, R, "mean")
    pb.softmax_bwd(sp, sdp, sdx, R, C, rowscale_const=1.0 / R)
    prog = HipProgram(ctx, pb.image())
    x = rng.standard_normal((R, C), dtype=np.float32) * 2
    mask = rng.random((R, C), dtype=np.float32) < 0.01
    x[mask] = 30.0
    bx, bdp = ctx.upload(x), ctx.upload(rng.standard_normal((R, C), dtype=np.float32))
    del x, mask
    bp, bl, bm, bdx = ctx.buffer(R * C * 4), ctx.buffer(R * 4), ctx.buffer(4), ctx.buffer(R * C * 4)
    prog.run([bx, bdp], [bp, bl, bm, bdx])
    prog.set_profiling(True)
    for _ in range(reps):
        prog.run([bx, bdp], [bp, bl, bm, bdx])
    t, runs = prog.step_times()
    fwd_ms, mean_ms, bwd_ms = (v / runs for v in t)
    fwd_bytes = R * C * 8 + R * 4
    bwd_bytes = R * C * 12
    out["c5_softmax_stress"] = {
        "shape": [R, C], "fwd_ms": round(fwd_ms, 4), "mean_ms": round(mean_ms, 4), "bwd_ms": round(bwd_ms, 4),
        "fwd_GBps": round(fwd_bytes / fwd_ms / 1e6, 1), "bwd_GBps": round(bwd_bytes / bwd_ms / 1e6, 1),
        "fwd_frac_hbm": round(fwd_bytes / fwd_ms / 1e6 / HBM_PEAK_GBS, 4),
        "bwd_frac_hbm": round(bwd_bytes / bwd_ms / 1e6 / HBM_PEAK_GBS, 4),
        "fwd_frac_copy": round(fwd_bytes / fwd_ms / 1e6 / copy_gbs, 4),
        "bwd_frac_copy": round(bwd_bytes / bwd_ms / 1e6 / copy_gbs, 4)}
    prog.close()
    for b in (bx, bdp, bp, bdx):
        b.close()
    # C2: single fused layer forward + backward, X [8192,1024] . W [1024,1024]
    B, I, O = 8192, 1024, 1024
    pb, outs = lower_dense_layer(B, I, O, "relu", "in_out")
    prog = HipProgram(ctx, pb.image())
    # X, dY ~ N(0,1); W Xavier-uniform (bound sqrt(6 / (in + out))); b zeros
    xb = float(np.sqrt(6.0 / (I + O)))
    ins = [ctx.upload(rng.standard_normal(B * I, dtype=np.float32)),
           ctx.upload(rng.uniform(-xb, xb, I * O).astype(np.float32)),
           ctx.upload(np.zeros(O, np.float32)),
           ctx.upload(rng.standard_normal(B * O, dtype=np.float32))]
    obs = [ctx.buffer(s.nbytes) for s in outs]
    for _ in range(5):
        prog.run(ins, obs)
    # the runtime's default launch mode (direct launches: every step is a large GEMM) with the
    # two-stream schedule, 100 synchronous calls
    t0 = time.perf_counter()
    for _ in range(100):
        prog.run(ins, obs)
    wall = (time.perf_counter() - t0) / 100 * 1e3
    # then a profiled pass (one stream, events per step) for the device-time breakdown
    prog.set_profiling(True)
    for _ in range(reps * 4):
        prog.run(ins, obs)
    t, runs = prog.step_times()
    dev = sum(t) / runs
    out["c2_fused_layer"] = {"ms": round(wall, 4), "TFLOPs": round(3 * 2 * B * I * O / wall / 1e9, 1),
                             "graph_replay": prog.graph_mode(),
                             "device_ms_profiled": round(dev, 4),
                             "steps_ms_profiled": [round(v / runs, 4) for v in t]}
    prog.close()
    out["c3_classifier_adam"] = c3_line(ctx, rng)
    # C1: 16 -> 64 -> 1 tanh MLP, MSE, SGD 0.01, batch 256 (builder weights, seed 0): the
    # 20-step run, launch-bound; the first run also captures the step's graph
    spec = MlpSpec.chain([16, 64, 1], hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 0, "builder")
    sess = HipTrainingSession.open(ctx, spec, Ws, bs, Sgd(0.01), 256)
    x1 = ctx.upload(rng.standard_normal((256, 16)).astype(np.float32))
    y1 = ctx.upload(rng.standard_normal((256, 1)).astype(np.float32))
    t0 = time.perf_counter()
    for _ in range(20):
        sess.run_resident(x1, y1)
    first = float(sess.objective())
    cold = time.perf_counter() - t0
    t0 = time.perf_counter()
    for _ in range(20 * reps):
        sess.run_resident(x1, y1)
    float(sess.objective())
    warm = (time.perf_counter() - t0) / reps
    out["c1_plumbing_mlp"] = {"ms_20_steps": round(warm * 1e3, 3),
                              "ms_20_steps_first": round(cold * 1e3, 3),
                              "us_per_step": round(warm / 20 * 1e6, 2), "objective_step20": first}
    sess.close()
    # Canonical host publication of the MLP-4096 output [4096, 4096] FLOAT32: dense and a
    # transposed view, device packing + one device-to-host copy into pageable host memory
    from synaptik_amd.backend import HipBackendIntegration, TensorDescriptor
    integ = HipBackendIntegration.open(0)
    data = rng.standard_normal((BATCH, WIDTH), dtype=np.float32)
    buf = integ.borrow("FLOAT32", data)
    pub = {}
    for name, desc in (("dense", TensorDescriptor("FLOAT32", (BATCH, WIDTH))),
                       ("transposed", TensorDescriptor("FLOAT32", (WIDTH, BATCH), (1, WIDTH)))):
        integ.copy_to_canonical_host_bytes(buf, desc, data.nbytes)
        t0 = time.perf_counter()
        for _ in range(reps):
            integ.copy_to_canonical_host_bytes(buf, desc, data.nbytes)
        ms = (time.perf_counter() - t0) / reps * 1e3
        pub[name] = {"ms": round(ms, 3), "host_GBps": round(data.nbytes / ms / 1e6, 1)}
    buf.download(np.float32)
    t0 = time.perf_counter()
    for _ in range(reps):
        buf.download(np.float32)
    raw_ms = (time.perf_counter() - t0) / reps * 1e3
    out["canonical_publication"] = {"shape": [BATCH, WIDTH], "dtype": "FLOAT32", **pub,
                                    "raw_download_ms": round(raw_ms, 3)}
    buf.close()
    integ.close()
    if cpu:
        add_cpu_baselines(out)
        from oracle import oracle
        raw = data[:256].tobytes()
        t0 = time.perf_counter()
        oracle.canonical_bytes(raw, 4, (256, WIDTH))
        dt = time.perf_counter() - t0
        out["canonical_publication"]["cpu_baseline"] = {
            "ms_full": round(dt * BATCH / 256 * 1e3, 1), **host_cores(), "kind": "port",
            "extrapolated": True,
            "sample": f"oracle per-element packing of 256 of 4096 rows ({dt:.3f} s), scaled x16"}
    return out


def host_cores() -> dict:
    """The host's core count (nproc: the CPUs this process may run on) beside the threads used."""
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count() or 1
    return {"cores": 1, "nproc": nproc}


def add_cpu_baselines(out: dict) -> None:
    """The oracle (1 thread) on the secondary configs: C1, C2 and C5 in full, C3 as one complete
    1024-row Adam step (each of its 50 steps is the same work)."""
    from oracle import oracle
    from synaptik_amd.training import MlpSpec, init_parameters
    rng = np.random.default_rng(8)
    # C1: the full 20-step run of 16 -> 64 -> 1 tanh, MSE, SGD 0.01, batch 256
    spec = MlpSpec.chain([16, 64, 1], hidden="tanh", loss="mse")
    Ws, bs = init_parameters(spec, 0, "builder")
    model = oracle.OracleMLP(Ws, bs, ["tanh", None], "mse", dict(kind="sgd", lr=0.01))
    x1 = rng.standard_normal((256, 16)).astype(np.float32)
    y1 = rng.standard_normal((256, 1)).astype(np.float32)
    t0 = time.perf_counter()
    for _ in range(20):
        model.step(x1, y1)
    dt = time.perf_counter() - t0
    if "c1_plumbing_mlp" in out:
        out["c1_plumbing_mlp"]["cpu_baseline"] = {
            "ms_20_steps": round(dt * 1e3, 3), **host_cores(), "kind": "port",
            "extrapolated": False, "sample": "the full 20-step run"}
    # C5: the full [65536, 4096] forward (softmax, LSE) and backward, in 8192-row chunks (the
    # oracle is row-wise, so the chunks do the same work as one call with a bounded footprint)
    rows, C, chunk = 65536, 4096, 8192
    dt = 0.0
    for r0 in range(0, rows, chunk):
        x = rng.standard_normal((chunk, C), dtype=np.float32) * 2
        g = rng.standard_normal((chunk, C), dtype=np.float32)
        t0 = time.perf_counter()
        p = oracle.softmax_rows(x)
        oracle.logsumexp_rows(x)
        oracle.softmax_grad_rows(p, g)
        dt += time.perf_counter() - t0
    del x, g, p
    gpu_ms = out["c5_softmax_stress"]["fwd_ms"] + out["c5_softmax_stress"]["bwd_ms"]
    out["c5_softmax_stress"]["cpu_baseline"] = {
        "rows_per_s": round(rows / dt, 1), "gpu_rows_per_s": round(65536 / (gpu_ms * 1e-3), 1),
        "ms_full": round(dt * 1e3, 1), **host_cores(), "kind": "port", "extrapolated": False,
        "sample": f"all 65536 rows of [65536,4096], fwd+bwd, in 8192-row chunks ({dt:.2f} s)"}
    # C2: the full layer, 8192 rows: forward + both backward GEMMs + db
    B, I, O = 8192, 1024, 1024
    X = rng.standard_normal((B, I), dtype=np.float32)
    W = rng.standard_normal((I, O), dtype=np.float32) * 0.05
    dY = rng.standard_normal((B, O), dtype=np.float32)
    t0 = time.perf_counter()
    Y = oracle.activation("relu", oracle.matmul(X, W))
    dZ = oracle.activation_grad("relu", dY, Y)
    oracle.matmul(dZ, W, trans_b=True)
    oracle.matmul(X, dZ, trans_a=True)
    oracle.colsum(dZ)
    dt = time.perf_counter() - t0
    out["c2_fused_layer"]["cpu_baseline"] = {
        "ms_full_layer": round(dt * 1e3, 1), **host_cores(), "kind": "port",
        "extrapolated": False, "sample": f"the full layer, {B} rows ({dt:.2f} s)"}
    # C3: one complete Adam step of the classifier on all 1024 rows
    spec = MlpSpec.chain([784, 1024, 1024, 10], hidden="relu", loss="ce")
    Ws, bs = init_parameters(spec, 0, "builder_he_normal")
    model = oracle.OracleMLP(Ws, bs, ["relu", "relu", None], "ce",
                             dict(kind="adam", lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8))
    xb = rng.uniform(0, 1, (1024, 784)).astype(np.float32)
    yb = rng.integers(0, 10, 1024)
    t0 = time.perf_counter()
    model.step(xb, yb)
    step_s = time.perf_counter() - t0
    out["c3_classifier_adam"]["cpu_baseline"] = {
        "samples_per_s": round(1024 / step_s, 1), "ms_per_step": round(step_s * 1e3, 1),
        **host_cores(), "kind": "port", "extrapolated": False,
        "sample": f"one complete step (1024 rows, fwd+bwd+Adam, {step_s:.2f} s) of the 50"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-sample", type=int, default=192, help="rows for the CPU baseline (0 = skip)")
    ap.add_argument("--no-secondary", action="store_true", help="skip the C2/C3/C5 lines")
    ap.add_argument("--probe", action="store_true",
                    help="counter probe: 3 launches each of one 4096^3 NT GEMM and a 256 MiB copy")
    ap.add_argument("--gemm-layouts", action="store_true",
                    help="plain GEMM TFLOP/s in the NT / NN / TN / TT layouts at three shapes")
    ap.add_argument("--c3-only", action="store_true",
                    help="only the C3 line (for kernel profiles of the classifier step)")
    ap.add_argument("--one-stream", action="store_true",
                    help="with --c3-only: run the step's program on one stream")
    ap.add_argument("--secondary-only", action="store_true",
                    help="only the C2/C3/C5 and publication lines, without CPU baselines "
                         "(for kernel profiles)")
    args = ap.parse_args()
    if args.probe:
        return probe()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this backend has no multi-GPU path "
              "(a data-parallel replica per GPU is the design); run with --gpus 1", file=sys.stderr)
        return 2

    from synaptik_amd.native import HipContext
    ctx = HipContext(0)
    if args.gemm_layouts:
        print(json.dumps({"gemm_layouts_TFLOPs": gemm_layouts(ctx)}), flush=True)
        ctx.close()
        return 0
    if args.c3_only:
        print(json.dumps({"c3_classifier_adam": c3_line(ctx, np.random.default_rng(7),
                                                        args.one_stream)}), flush=True)
        ctx.close()
        return 0
    if args.secondary_only:
        print(json.dumps({"secondary": secondary(ctx, cpu=False)}), flush=True)
        ctx.close()
        return 0
    info = ctx.device_info()
    spec, Ws, bs, sess, x, y = build_session(ctx)
    print(f"[bench] device {info}", file=sys.stderr, flush=True)

    for _ in range(args.warmup):
        sess.run_resident(x, y)
    prog = sess.program
    prog.set_profiling(True)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        sess.run_resident(x, y)
    elapsed = time.perf_counter() - t0
    step_ms, runs = prog.step_times()
    prog.set_profiling(False)
    loss = float(sess.objective())
    if not np.isfinite(loss):
        print(f"[bench] non-finite objective {loss}", file=sys.stderr)
        return 1

    from synaptik_amd.program import OP_GEMM, OP_OPTIMIZER, OP_COLSUM, OP_MSE
    import struct
    # classify steps by re-lowering the same program (step order is deterministic)
    from synaptik_amd.training import Sgd, lower_training_step
    pb, _ = lower_training_step(spec, BATCH, Sgd(LR, momentum=MOMENTUM))
    ops = [st.opcode for st in pb.steps]
    per = {}
    for op, ms in zip(ops, step_ms):
        per.setdefault(op, []).append(ms / runs)
    gemm_ms = per.get(OP_GEMM, [])
    avg_gemm_ms = sum(gemm_ms) / len(gemm_ms)
    achieved = gemm_flops() / (avg_gemm_ms * 1e-3) / 1e12
    ms_per_step = elapsed / args.steps * 1e3
    opt_ms = sum(per.get(OP_OPTIMIZER, []))
    breakdown = {
        "gemm_ms_per_step": round(sum(gemm_ms), 4),
        "optimizer_ms_per_step": round(opt_ms, 4),
        "colsum_ms_per_step": round(sum(per.get(OP_COLSUM, [])), 4),
        "mse_ms_per_step": round(sum(per.get(OP_MSE, [])), 4),
        "device_ms_per_step": round(sum(step_ms) / runs, 4),
    }
    # The weights' updates run in the dW GEMM epilogues; the streaming optimizer pass covers the
    # biases only (one staged pass reads p, g, m and writes the candidate p, m: 20 B each).
    n_bias = sum(layer.fan_out for layer in spec.layers if layer.bias)
    opt_gbs = (20.0 * n_bias) / (opt_ms * 1e-3) / 1e9 if opt_ms > 0 else 0.0
    print(f"[bench] breakdown {breakdown}; bias optimizer pass {opt_gbs:.0f} GB/s "
          f"({n_bias} parameters, launch-bound)", file=sys.stderr, flush=True)

    # The same step with the batch handed over as host arrays (upload over PCIe from pageable
    # memory, objective downloaded): a reported figure, never `value`.
    rng = np.random.default_rng(3)
    xh = rng.standard_normal((BATCH, WIDTH), dtype=np.float32)
    yh = rng.standard_normal((BATCH, WIDTH), dtype=np.float32)
    sess.run(xh, yh)
    t0 = time.perf_counter()
    host_steps = 5
    for _ in range(host_steps):
        sess.run(xh, yh)
    host_ms = (time.perf_counter() - t0) / host_steps * 1e3
    host_batch = {"samples_per_s": round(BATCH / host_ms * 1e3, 1), "ms_per_step": round(host_ms, 3),
                  "note": "batch uploaded from pageable host memory each step (2 x 64 MiB)"}
    # The same host batches through run_pipelined: batch i+1 goes through the pinned staging ring
    # on the copy stream while step i runs (objective downloaded every step).
    xh2 = rng.standard_normal((BATCH, WIDTH), dtype=np.float32)
    yh2 = rng.standard_normal((BATCH, WIDTH), dtype=np.float32)
    pipe_batches = [(xh, yh), (xh2, yh2)] * 6
    sess.run_pipelined(pipe_batches[:2])
    t0 = time.perf_counter()
    sess.run_pipelined(pipe_batches)
    pipe_ms = (time.perf_counter() - t0) / len(pipe_batches) * 1e3
    host_pipe = {"samples_per_s": round(BATCH / pipe_ms * 1e3, 1), "ms_per_step": round(pipe_ms, 3),
                 "note": "12 host batches from pageable memory, each staged on the copy stream "
                         "while the previous step runs (run_pipelined); the first batch's upload "
                         "is not overlapped and is included"}
    sess.close()
    extra = None if args.no_secondary else secondary(ctx, cpu=args.cpu_sample > 0)
    if extra is not None:
        extra["c4_host_batch"] = host_batch
        extra["c4_host_batch_pipelined"] = host_pipe
    if extra:
        print(f"[bench] secondary {extra}", file=sys.stderr, flush=True)
    cpu = None
    if args.cpu_sample > 0:
        cpu = cpu_baseline(args.cpu_sample)
        # the OpenBLAS route on one thread (as the reference qualifies it) and on the host's share
        # of cores (16 per GPU on the benchmark boxes)
        share = min(16, os.cpu_count() or 1)
        cpu["openblas_route"] = [openblas_baseline(1, 256), openblas_baseline(share, 1024)]
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)

    result = {
        "metric": "training samples/sec at 1 MI355X (MLP-4096) + GEMM % of fp32 MFMA peak",
        "value": round(BATCH * args.steps / elapsed, 1),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "MLP-4096 training step (benchmark configuration C4, configs[3])",
                   "layers": "4096->4096x4 hidden->4096 ReLU", "global_batch": BATCH,
                   "loss": "MSE mean", "optimizer": f"SGD lr={LR} momentum={MOMENTUM}",
                   "parallelism": "single GPU", "objective_after": loss},
        "roofline": {"bound": "mfma", "kernel": "gemm_f32_v2 (14 per step, 4096^3 each)",
                     "achieved": round(achieved, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": measured_gemm_traffic()},
        "breakdown": breakdown,
        "cpu_baseline": cpu,
        "secondary": extra,
    }
    print(json.dumps(result), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
