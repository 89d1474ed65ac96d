"""Benchmark of the plugin's hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--cpu-seconds S]

Headline (BASELINE.json metric): int4 group-64 dequant-matmul at M=16,
K=4096, N=14336, bf16 out -- `value` is its algorithmic HBM throughput in
GB/s over K timed steps (one step = one kernel call on one of several
rotating input sets whose total exceeds the 256 MB Infinity Cache, inputs
resident in HBM).  The steps are captured in HIP graphs so host launch cost
is not timed; HIP events bracket the timed region on the launch stream.

Printed: ONE JSON line with the headline, its roofline object, the CPU
baseline (the oracle's C port of the same computation on the host cores,
kind "port"), and `secondary` entries for the other hot-path kernels.
"""

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (REPO, os.path.join(REPO, "jax-metallib_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0

METRIC = "int4 dequant-matmul GB/s (% HBM peak) at M=16; bf16 GEMM TFLOP/s (% MFMA peak)"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def int4_bytes(M, K, N):
    """Algorithmic HBM bytes of one int4 g64 call: W + bf16 scales + uint8
    zero-points + bf16 x + bf16 y."""
    return K // 2 * N + (K // 64) * N * 2 + (K // 64) * N + M * K * 2 + M * N * 2


def int8_bytes(M, K, N):
    return K * N + N * 4 + M * K * 2 + M * N * 2


def time_graph_launches(torch, fn, nsets, steps, warmup):
    """Run fn(i) for i in range(steps) (set = i % nsets) inside HIP graphs and
    return (elapsed seconds for `steps` calls, calls) measured by events on
    the launch stream."""
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(max(warmup, nsets)):
            fn(i % nsets)
    torch.cuda.synchronize()
    # One graph of up to 1000 back-to-back calls, replayed: each replay's
    # launch costs a few microseconds, which 50-call graphs spread at about
    # 0.2 us over a 13 us call.
    chunk = min(steps, max(nsets, 1000))
    chunk -= chunk % nsets if chunk > nsets else 0
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for i in range(chunk):
            fn(i % nsets)
    reps, rem = divmod(steps, chunk)
    g_rem = None
    if rem:
        g_rem = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_rem, stream=stream):
            for i in range(rem):
                fn(i % nsets)
    # graph warmup replay
    g.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(reps):
            g.replay()
        if g_rem is not None:
            g_rem.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3, steps


def bench_int4(torch, ops, steps, warmup, M=16, K=4096, N=14336):
    from mi355x import synthetic

    per_set = int4_bytes(M, K, N)
    nsets = max(2, -(-300 * 2 ** 20 // per_set))  # > 256 MB Infinity Cache
    rng = np.random.default_rng(0)
    sets = []
    for _ in range(nsets):
        x, packed, s, z = synthetic.int4_case(rng, M, K, N)
        sets.append((
            torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda(),
            torch.from_numpy(packed).cuda(),
            torch.from_numpy(s.view(np.int16)).view(torch.bfloat16).cuda(),
            torch.from_numpy(z).cuda(),
            torch.empty((M, N), dtype=torch.bfloat16, device="cuda"),
        ))

    def fn(i):
        x, w, s, z, y = sets[i]
        ops.int4_g64_matmul(x, w, s, z, out=y)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    t = secs / n
    return {"bytes": per_set, "sec_per_call": t, "gbs": per_set / t / 1e9, "nsets": nsets,
            "flops": 2 * M * K * N}


def bench_int8(torch, ops, steps, warmup, M=16, K=4096, N=14336):
    from mi355x import synthetic

    per_set = int8_bytes(M, K, N)
    nsets = max(2, -(-300 * 2 ** 20 // per_set))
    rng = np.random.default_rng(0)
    sets = []
    for _ in range(nsets):
        x, w, s = synthetic.int8_case(rng, M, K, N)
        sets.append((
            torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).cuda(),
            torch.from_numpy(w).cuda(), torch.from_numpy(s).cuda(),
            torch.empty((M, N), dtype=torch.bfloat16, device="cuda"),
        ))

    def fn(i):
        x, w, s, y = sets[i]
        ops.int8_pc_matmul(x, w, s, out=y)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    t = secs / n
    return {"bytes": per_set, "sec_per_call": t, "gbs": per_set / t / 1e9, "nsets": nsets}


def bench_decoder(torch, reps=10):
    """The workload's Llama-style decoder (4 layers, hidden 2048, 16 x 128
    heads, SwiGLU 8192, batch 4 x seq 2048, int4 g64 weights, random init):
    one forward captured in a HIP graph, replayed `reps` times."""
    from mi355x import decoder

    cfg = decoder.DecoderConfig()
    weights = decoder.init_weights(cfg, seed=0)
    cos, sin = decoder.rope_tables(cfg)
    buf = decoder.Buffers(cfg)
    x0 = (torch.randn((cfg.tokens, cfg.hidden), device="cuda", generator=torch.Generator("cuda").manual_seed(0))
          .to(torch.bfloat16))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        buf.x.copy_(x0)
        decoder.forward(cfg, weights, buf, cos, sin)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        decoder.forward(cfg, weights, buf, cos, sin)
    g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / reps
    return {"ms": ms, "tokens_per_s": cfg.tokens / ms * 1e3, "tflops": cfg.matmul_flops() / ms / 1e9,
            "config": {"layers": cfg.layers, "hidden": cfg.hidden, "heads": cfg.heads, "head_dim": cfg.head_dim,
                       "ffn": cfg.ffn, "batch": cfg.batch, "seq": cfg.seq, "weights": "int4 g64, random init",
                       "data": "synthetic", "flops_counted": "projections + causal attention products"}}


def _rot_sets(total_bytes_per_set, floor_sets=2):
    """How many distinct input sets to rotate so their total exceeds the
    256 MB Infinity Cache."""
    return max(floor_sets, -(-300 * 2 ** 20 // total_bytes_per_set))


def bench_gemm_bf16(torch, ops, steps, warmup, batch=1, M=4096, N=4096, K=4096, out_f32=False):
    per = 2 * batch * (M * K + K * N)
    nsets = _rot_sets(per)
    g = torch.Generator(device="cuda").manual_seed(0)
    sc = 1.0 / np.sqrt(np.sqrt(K))
    sets = []
    for _ in range(nsets):
        a = (torch.randn((batch, M, K), device="cuda", generator=g) * sc).to(torch.bfloat16)
        b = (torch.randn((batch, K, N), device="cuda", generator=g) * sc).to(torch.bfloat16)
        c = torch.empty((batch, M, N), dtype=torch.float32 if out_f32 else torch.bfloat16, device="cuda")
        sets.append((a, b, c))

    def fn(i):
        a, b, c = sets[i]
        ops.gemm_bf16(a, b, out_f32=out_f32, out=c)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    t = secs / n
    flops = 2.0 * batch * M * N * K
    out_bytes = batch * M * N * (4 if out_f32 else 2)
    return {"sec_per_call": t, "tflops": flops / t / 1e12, "bytes": per + out_bytes, "nsets": nsets}


def bench_torch_matmul(torch, steps, warmup, M=4096, N=4096, K=4096):
    """torch.matmul (hipBLASLt on ROCm) on the same shape and distribution,
    timed the same way: the vendor library's figure on this box."""
    per = 2 * (M * K + K * N)
    nsets = _rot_sets(per)
    g = torch.Generator(device="cuda").manual_seed(0)
    sc = 1.0 / np.sqrt(np.sqrt(K))
    sets = [((torch.randn((M, K), device="cuda", generator=g) * sc).to(torch.bfloat16),
             (torch.randn((K, N), device="cuda", generator=g) * sc).to(torch.bfloat16),
             torch.empty((M, N), dtype=torch.bfloat16, device="cuda")) for _ in range(nsets)]

    def fn(i):
        a, b, c = sets[i]
        torch.matmul(a, b, out=c)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    return 2.0 * M * N * K / (secs / n) / 1e12


def bench_gemm_f32(torch, ops, steps, warmup, M=2048, N=2048, K=2048):
    per = 4 * (M * K + K * N)
    nsets = _rot_sets(per)
    g = torch.Generator(device="cuda").manual_seed(0)
    sets = [((torch.randn((M, K), device="cuda", generator=g)), torch.randn((K, N), device="cuda", generator=g),
             torch.empty((M, N), device="cuda")) for _ in range(nsets)]

    def fn(i):
        a, b, c = sets[i]
        ops.gemm_f32(a, b, out=c)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    t = secs / n
    return {"sec_per_call": t, "tflops": 2.0 * M * N * K / t / 1e12}


def bench_rowop(torch, ops, kind, dtype, steps, warmup, rows=8192, cols=8192):
    """softmax / rmsnorm / argmax / chain6 on X [rows, cols] ~ N(0, 2)."""
    tdt = torch.float32 if dtype == "f32" else torch.bfloat16
    esz = 4 if dtype == "f32" else 2
    per = rows * cols * esz
    nsets = _rot_sets(per)
    g = torch.Generator(device="cuda").manual_seed(0)
    xs = [(torch.randn((rows, cols), device="cuda", generator=g) * np.sqrt(2.0)).to(tdt) for _ in range(nsets)]
    gam = (torch.rand((cols,), device="cuda", generator=g) + 0.5).to(tdt)
    if kind == "argmax":
        out = torch.empty((rows,), dtype=torch.int32, device="cuda")
        moved = per + rows * 4
    else:
        out = torch.empty((rows, cols), dtype=tdt, device="cuda")
        moved = 2 * per + (cols * esz if kind == "rmsnorm" else 0)
    def fn(i):
        x = xs[i]
        if kind == "softmax":
            ops.softmax(x, out=out)
        elif kind == "rmsnorm":
            ops.rmsnorm(x, gam, out=out)
        elif kind == "argmax":
            ops.argmax(x, out=out)
        else:
            ops.elementwise(CHAIN6, [x], out_slot=8, out=out)

    secs, n = time_graph_launches(torch, fn, nsets, steps, warmup)
    t = secs / n
    return {"sec_per_call": t, "gbs": moved / t / 1e9, "bytes": moved}


def _hbm_entry(gbs, us, extra=None, profile=None):
    """A secondary HBM-bound line; `profile` names the committed counter
    summary (profiles/<profile>_traffic.md) its roofline.traffic comes from."""
    traffic, note = traffic_from_profiles(profile) if profile else (None, "no traffic profile")
    e = {"value": round(gbs, 2), "unit": "GB/s", "us_per_call": round(us, 3),
         "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_note": note}}
    if extra:
        e.update(extra)
    return e


def sources_digest(paths):
    """sha256 (16 hex digits) of the kernel sources a measurement was taken
    with, paths relative to the repository root."""
    import hashlib

    h = hashlib.sha256()
    for rel in paths:
        with open(os.path.join(REPO, rel), "rb") as f:
            h.update(rel.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


def traffic_from_profiles(kernel):
    """Measured HBM bytes per launch of `kernel`, from the committed rocprof
    PMC summary profiles/<kernel>_traffic.md (FETCH_SIZE + WRITE_SIZE per
    dispatch, scaled by the copy-kernel calibration it records).  The file
    names the kernel sources it was measured with and their digest; when the
    sources have changed since, the figure belongs to another kernel and None
    is returned.  Returns (bytes or None, note)."""
    path = os.path.join(REPO, "profiles", f"{kernel}_traffic.md")
    value, sources, digest = None, None, None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    value = int(line.split(":", 1)[1].strip())
                elif line.startswith("sources:"):
                    sources = line.split(":", 1)[1].split()
                elif line.startswith("sources_sha256:"):
                    digest = line.split(":", 1)[1].strip()
    except OSError:
        return None, "no traffic profile"
    if value is None or not sources or not digest:
        return None, "traffic profile without a source digest"
    try:
        now = sources_digest(sources)
    except OSError:
        return None, "traffic profile names missing sources"
    if now != digest:
        return None, f"stale: measured with sources {digest}, current {now}"
    return value, f"measured with sources {digest} (current)"


# The 6-op elementwise chain of the row-op lines: select(x > 0, max(log1p(exp(1.5 x + 0.5)), x), 1.5 x + 0.5).
CHAIN6 = [("LOAD", 0, 0, 0, 0, 0.0), ("CONST", 1, 0, 0, 0, 1.5), ("MUL", 2, 0, 1, 0, 0.0),
          ("CONST", 1, 0, 0, 0, 0.5), ("ADD", 3, 2, 1, 0, 0.0), ("EXP", 4, 3, 0, 0, 0.0),
          ("LOG1P", 5, 4, 0, 0, 0.0), ("MAX", 6, 5, 0, 0, 0.0), ("CONST", 1, 0, 0, 0, 0.0),
          ("CMP_GT", 7, 0, 1, 0, 0.0), ("SELECT", 8, 7, 6, 3, 0.0)]

PROFILE_KINDS = ("int4", "int8", "gemm", "gemm_f32", "qgemm", "qgemm8", "int4_m1", "int8_m1", "int4_shard",
                 "int8_shard", "bmm", "dequant4096", "dequant4096_8", "attention", "softmax_f32", "softmax_bf16",
                 "rmsnorm_f32", "rmsnorm_bf16", "argmax_f32", "argmax_bf16", "chain6_f32", "chain6_bf16")


def _profile_case(torch, ops, kind):
    """One input set of a bench line's workload, resident on the device, and
    the call that runs it once (eagerly, on the current stream)."""
    from mi355x import synthetic

    def bf(a):
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()

    rng = np.random.default_rng(0)
    g = torch.Generator(device="cuda").manual_seed(0)
    quant = {"int4": (16, 14336), "qgemm": (256, 14336), "int4_m1": (1, 14336), "int4_shard": (16, 1792),
             "dequant4096": (4096, 14336)}
    if kind in quant:
        M, N = quant[kind]
        x, packed, s, z = synthetic.int4_case(rng, M, 4096, N)
        xd, wd, sd, zd = bf(x), torch.from_numpy(packed).cuda(), bf(s), torch.from_numpy(z).cuda()
        yd = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        return lambda: ops.int4_g64_matmul(xd, wd, sd, zd, out=yd)
    if kind in ("int8", "int8_m1", "int8_shard", "qgemm8", "dequant4096_8"):
        M, N = {"int8": (16, 14336), "int8_m1": (1, 14336), "int8_shard": (16, 1792), "qgemm8": (256, 14336),
                "dequant4096_8": (4096, 14336)}[kind]
        x, w8, s8 = synthetic.int8_case(rng, M, 4096, N)
        xd, wd, sd = bf(x), torch.from_numpy(w8).cuda(), torch.from_numpy(s8).cuda()
        yd = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        return lambda: ops.int8_pc_matmul(xd, wd, sd, out=yd)
    if kind in ("gemm", "bmm"):
        batch, M, N, K = (1, 4096, 4096, 4096) if kind == "gemm" else (16, 2048, 2048, 128)
        sc = 1.0 / np.sqrt(np.sqrt(K))
        a = (torch.randn((batch, M, K), device="cuda", generator=g) * sc).to(torch.bfloat16)
        b = (torch.randn((batch, K, N), device="cuda", generator=g) * sc).to(torch.bfloat16)
        c = torch.empty((batch, M, N), dtype=torch.bfloat16, device="cuda")
        if kind == "gemm":
            a, b, c = a[0], b[0], c[0]
        return lambda: ops.gemm_bf16(a, b, out=c)
    if kind == "gemm_f32":
        a = torch.randn((2048, 2048), device="cuda", generator=g)
        b = torch.randn((2048, 2048), device="cuda", generator=g)
        c = torch.empty((2048, 2048), device="cuda")
        return lambda: ops.gemm_f32(a, b, out=c)
    if kind == "attention":
        # The decoder's attention at the workload's shape: 4 x 16 heads of
        # 2048 positions x 128, causal, heads merged on output.
        B, H, S, D = 4, 16, 2048, 128
        q, k, v = [torch.randn((B * H, S, D), device="cuda", generator=g).to(torch.bfloat16) for _ in range(3)]
        o = torch.empty((B * S, H * D), dtype=torch.bfloat16, device="cuda")
        return lambda: ops.attention_causal(q, k, v, B, H, 1.0 / np.sqrt(D), out=o)
    op, dt = kind.rsplit("_", 1)
    tdt = torch.float32 if dt == "f32" else torch.bfloat16
    x = (torch.randn((8192, 8192), device="cuda", generator=g) * np.sqrt(2.0)).to(tdt)
    gam = (torch.rand((8192,), device="cuda", generator=g) + 0.5).to(tdt)
    if op == "argmax":
        out = torch.empty((8192,), dtype=torch.int32, device="cuda")
        return lambda: ops.argmax(x, out=out)
    out = torch.empty_like(x)
    if op == "softmax":
        return lambda: ops.softmax(x, out=out)
    if op == "rmsnorm":
        return lambda: ops.rmsnorm(x, gam, out=out)
    return lambda: ops.elementwise(CHAIN6, [x], out_slot=8, out=out)


def profile_run(torch, ops, kinds, steps):
    """Eager (no graph) launches of each listed workload in turn (5 warm-up
    calls + `steps` timed ones, one input set each), for rocprofv3 --pmc and
    kernel-trace runs, followed by a plain 256 MiB device copy (8 times) that
    calibrates FETCH_SIZE and WRITE_SIZE.  Returns {kind: seconds per call}
    (HIP events on the launch stream)."""
    times = {}
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for kind in kinds:
            if kind not in PROFILE_KINDS:
                raise SystemExit(f"bench.py: unknown --profile kind {kind} (one of {', '.join(PROFILE_KINDS)})")
            # A one-thread spin kernel marks where this workload's
            # dispatches begin in the profiler's dispatch-ordered output.
            torch.cuda._sleep(100)
            fn = _profile_case(torch, ops, kind)
            for _ in range(5):
                fn()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            for _ in range(steps):
                fn()
            end.record(stream)
            torch.cuda.synchronize()
            times[kind] = start.elapsed_time(end) / 1e3 / steps
            print(f"[profile] {kind}: {times[kind] * 1e6:.3f} us per call", flush=True)
            del fn
            torch.cuda.empty_cache()
        src = torch.empty(256 * 2 ** 20, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
    return times


def profile_layer(steps):
    """One decoder layer (4 x 2048 tokens) compiled from its StableHLO and
    executed `steps` times through the runtime (execute + await each), for
    rocprofv3 kernel traces of the compiled path.  Returns seconds per call."""
    from mi355x import programs, runtime, synthetic

    client = runtime.Client()
    try:
        x, w, cos, sin = synthetic.decoder_layer_case(np.random.default_rng(0), 4, 2048, 2048, 16, 128, 8192)
        exe = client.compile(programs.decoder_layer(4, 2048, 2048, 16, 128, 8192))
        bufs = [client.buffer(a, runtime.BF16) if is_bf16 else client.buffer(a)
                for a, is_bf16 in synthetic.decoder_layer_arguments(x, w, cos, sin)]
        times = []
        for i in range(steps + 2):
            t0 = time.perf_counter()
            outs, done = exe.execute(bufs)
            done.wait()
            if i >= 2:
                times.append(time.perf_counter() - t0)
            for o in outs:
                o.close()
        for b in bufs:
            b.close()
        exe.close()
    finally:
        client.close()
    times.sort()
    return times[len(times) // 2]


def available_cores():
    """Cores this process may run on: the affinity mask, further limited by a
    cgroup CPU quota when one is set (cpu.max: quota period)."""
    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota, period = f.read().split()[:2]
        if quota != "max":
            cores = max(1, min(cores, int(int(quota) // int(period))))
    except (OSError, ValueError):
        pass
    return cores


def cpu_baseline_qmm(fmt, target_s, M=16, K=4096, N=14336, unit="GB/s"):
    """Time the oracle's C port of the int4 g64 / int8 per-channel matmul
    (OpenMP, every available core) on a column slice of the [M, K] x [K, N]
    case, sized to roughly target_s seconds; report the GPU line's unit:
    GB/s of its algorithmic bytes per processed column, or TFLOP/s."""
    from oracle import cport, quant

    cores = available_cores()
    cport.threads(cores)
    rng = np.random.default_rng(0)
    if fmt == "int4":
        args = quant.make_int4_case(rng, M, K, N)
        call, nbytes = cport.int4_g64_matmul, int4_bytes(M, K, N)
    else:
        args = quant.make_int8_case(rng, M, K, N)
        call, nbytes = cport.int8_pc_matmul, int8_bytes(M, K, N)
    ncols = 64
    t0 = time.perf_counter()
    call(*args, n_range=(0, ncols))
    t1 = time.perf_counter() - t0
    ncols = int(min(N, max(64, ncols * target_s / max(t1, 1e-6))))
    ncols -= ncols % 64
    ncols = max(ncols, 64)
    reps = 0
    t0 = time.perf_counter()
    while True:
        call(*args, n_range=(0, ncols))
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    per_call = el / reps
    if unit == "GB/s":
        value = nbytes * (ncols / N) / per_call / 1e9
    else:
        value = 2.0 * M * K * ncols / per_call / 1e12
    name = "int4 g64" if fmt == "int4" else "int8 per-channel"
    return {"value": round(value, 4 if unit != "GB/s" else 3), "unit": unit, "cores": cores, "kind": "port",
            "sample": f"oracle/c {name} M={M} K={K}, columns [0,{ncols}) of N={N}, "
                      f"{reps} run(s), {el:.1f}s, OpenMP threads={cores}"}


def cpu_baseline_int4(target_s, M=16, K=4096, N=14336):
    """The headline's CPU baseline: cpu_baseline_qmm for int4 g64 in GB/s."""
    return cpu_baseline_qmm("int4", target_s, M, K, N)


def cpu_baseline_bmm(target_s, batch=16, M=2048, K=128, N=2048):
    """The C port's bf16 GEMM on a row slice of one batch of the batched
    product; GB/s of the GPU line's algorithmic bytes (A + B + C) per
    processed output row."""
    from oracle import cport
    from oracle.bf16 import f32_to_bf16_bits

    cores = available_cores()
    cport.threads(cores)
    rng = np.random.default_rng(0)
    a = f32_to_bf16_bits(rng.standard_normal((M, K)).astype(np.float32))
    b = f32_to_bf16_bits(rng.standard_normal((K, N)).astype(np.float32))
    rows = cores
    t0 = time.perf_counter()
    cport.gemm_bf16(a, b, m_range=(0, rows))
    t1 = time.perf_counter() - t0
    rows = int(min(M, max(cores, rows * target_s / max(t1, 1e-6))))
    reps, t0 = 0, time.perf_counter()
    while True:
        cport.gemm_bf16(a, b, m_range=(0, rows))
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    line_bytes = batch * (M * K + K * N + M * N) * 2
    gbs = line_bytes * rows / (batch * M) / (el / reps) / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle/c bf16 GEMM [{M},{K}] x [{K},{N}] (one of {batch} batches), rows [0,{rows}), "
                      f"{reps} run(s), {el:.1f}s, OpenMP threads={cores}"}


def cpu_baseline_gemm_f32(target_s, n=2048):
    """The C port's f32 GEMM on a row slice of the n^3 product; TFLOP/s."""
    from oracle import cport

    cores = available_cores()
    cport.threads(cores)
    rng = np.random.default_rng(0)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    rows = cores
    t0 = time.perf_counter()
    cport.gemm_f32(a, b, m_range=(0, rows))
    t1 = time.perf_counter() - t0
    rows = int(min(n, max(cores, rows * target_s / max(t1, 1e-6))))
    reps, t0 = 0, time.perf_counter()
    while True:
        cport.gemm_f32(a, b, m_range=(0, rows))
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    tflops = 2.0 * rows * n * n / (el / reps) / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle/c f32 GEMM K={n} N={n}, rows [0,{rows}) of M={n}, {reps} run(s), {el:.1f}s, "
                      f"OpenMP threads={cores}"}


def cpu_baseline_decoder(layers=4, S=2048, hidden=2048, heads=16, head_dim=128, ffn=8192):
    """The decoder oracle (oracle/decoder.py: float64 numpy, bf16 roundings
    where the plugin writes bf16) on one layer of one S-token sequence, every
    position; tokens/s of the `layers`-layer forward (each token passes every
    layer).  A single timed call: it takes seconds."""
    from mi355x import synthetic
    from oracle import decoder as odec
    from oracle.bf16 import bf16_bits_to_f32

    cores = available_cores()
    rng = np.random.default_rng(0)
    x, w, _, _ = synthetic.decoder_layer_case(rng, 1, S, hidden, heads, head_dim, ffn)
    x0 = bf16_bits_to_f32(x).reshape(S, hidden)
    t0 = time.perf_counter()
    odec.layer_rows(x0, np.arange(S), w, heads, head_dim)
    el = time.perf_counter() - t0
    return {"value": round(S / (el * layers), 2), "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"oracle/decoder.py (float64 numpy, BLAS threads as the host sets them) one layer of one "
                      f"{S}-token sequence, {el:.1f}s, scaled to {layers} layers"}


def cpu_baseline_gemm(target_s, M=4096, K=4096, N=4096):
    """The oracle's C port of the bf16 GEMM (f32 accumulation, OpenMP over
    rows, every available core) on a row slice of the 4096^3 headline GEMM,
    sized to roughly target_s seconds; TFLOP/s of the slice."""
    from oracle import cport
    from oracle.bf16 import f32_to_bf16_bits

    cores = available_cores()
    cport.threads(cores)
    rng = np.random.default_rng(0)
    sc = 1.0 / np.sqrt(np.sqrt(K))
    a = f32_to_bf16_bits((rng.standard_normal((M, K)) * sc).astype(np.float32))
    b = f32_to_bf16_bits((rng.standard_normal((K, N)) * sc).astype(np.float32))
    rows = cores
    t0 = time.perf_counter()
    cport.gemm_bf16(a, b, m_range=(0, rows))
    t1 = time.perf_counter() - t0
    rows = int(min(M, max(cores, rows * target_s / max(t1, 1e-6))))
    reps, t0 = 0, time.perf_counter()
    while True:
        cport.gemm_bf16(a, b, m_range=(0, rows))
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    tflops = 2.0 * rows * K * N / (el / reps) / 1e12
    return {"value": round(tflops, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle/c bf16 GEMM K={K} N={N}, rows [0,{rows}) of M={M}, {reps} run(s), {el:.1f}s, "
                      f"OpenMP threads={cores}"}


_CPU_ROWS_X = {}


def _cpu_rows_input(dtype, rows, cols):
    """X [rows, cols] ~ N(0, 2) on the host (f32, or bf16 bits), made once."""
    key = (dtype, rows, cols)
    if key not in _CPU_ROWS_X:
        from mi355x import synthetic
        x = (np.random.default_rng(0).standard_normal((rows, cols), dtype=np.float32) * np.float32(np.sqrt(2.0)))
        _CPU_ROWS_X[key] = x if dtype == "f32" else synthetic.bf16_bits(x)
    return _CPU_ROWS_X[key]


def cpu_baseline_rowop(kind, dtype, target_s, rows=8192, cols=8192):
    """The oracle's C port of softmax / RMSNorm / argmax / the 6-op chain
    (OpenMP, every available core) on a row prefix of the 8192^2 case, sized
    to roughly target_s seconds; GB/s of the GPU line's algorithmic bytes per
    row (read + write, or read + the int32 index for argmax)."""
    from oracle import cport

    cores = available_cores()
    cport.threads(cores)
    x = _cpu_rows_input(dtype, rows, cols)
    esz = 4 if dtype == "f32" else 2
    g = np.random.default_rng(1).uniform(0.5, 1.5, cols).astype(np.float32)
    if dtype == "bf16":
        from oracle.bf16 import f32_to_bf16_bits
        g = f32_to_bf16_bits(g)
    per_row = cols * esz + 4 if kind == "argmax" else 2 * cols * esz

    def run(r):
        if kind == "softmax":
            cport.softmax(x[:r])
        elif kind == "rmsnorm":
            cport.rmsnorm(x[:r], g)
        elif kind == "argmax":
            (cport.argmax_f32 if dtype == "f32" else cport.argmax_bf16)(x[:r])
        else:
            cport.chain6(x[:r])

    r = 64
    t0 = time.perf_counter()
    run(r)
    t1 = time.perf_counter() - t0
    r = int(min(rows, max(64, r * (target_s / 4) / max(t1, 1e-6))))
    reps, t0 = 0, time.perf_counter()
    while True:
        run(r)
        reps += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    gbs = per_row * r / (el / reps) / 1e9
    return {"value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle/c {kind} {dtype}, rows [0,{r}) of {rows}x{cols}, {reps} run(s), {el:.1f}s, "
                      f"OpenMP threads={cores}"}


def cpu_baseline_plumbing(target_s, n=1024):
    """The oracle's C port of tanh(A @ B).sum(axis=1) on f32 [n, n] (OpenMP
    over rows, every available core): median microseconds per whole call."""
    from oracle import cport

    cores = available_cores()
    cport.threads(cores)
    rng = np.random.default_rng(0)
    a = rng.standard_normal((n, n)).astype(np.float32)
    b = rng.standard_normal((n, n)).astype(np.float32)
    times, t_end = [], time.perf_counter() + target_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        cport.plumbing(a, b)
        times.append(time.perf_counter() - t0)
    times.sort()
    return {"value": round(times[len(times) // 2] * 1e6, 1), "unit": "us/call", "cores": cores, "kind": "port",
            "sample": f"oracle/c plumbing n={n}, all rows, {len(times)} call(s), median, OpenMP threads={cores}"}


def bench_end_to_end(warmup=10, iters=50):
    """The plugin path as jax drives it: compile the workload's StableHLO
    once, then execute + await the completion event per call, with the inputs
    already in device buffers (the reference's method, benchmarks/vs_cpu.py:
    39-60: 1 compile, 10 warmups, 50 timed calls, median).  Reported apart
    from kernel time: it includes the host-side launch, the output buffer
    allocation and the completion wait."""
    from mi355x import programs, runtime, synthetic

    out = {}
    client = runtime.Client()
    try:
        rng = np.random.default_rng(0)
        x, packed, s, z = synthetic.int4_case(rng, 16, 4096, 14336)
        a = (rng.standard_normal((4096, 4096)) / 8).astype(np.float32)
        f32_to_bf16_bits = synthetic.bf16_bits
        pa = rng.standard_normal((1024, 1024)).astype(np.float32)
        pb = rng.standard_normal((1024, 1024)).astype(np.float32)
        cases = {
            "plumbing_tanh_matmul_sum_1024": (programs.plumbing(1024), [(pa, None), (pb, None)]),
            "int4_g64_M16_K4096_N14336": (programs.int4_g64_matmul(16, 4096, 14336),
                                          [(x, runtime.BF16), (packed, None), (s, runtime.BF16), (z, None)]),
            "bf16_gemm_4096": (programs.matmul(4096, 4096, 4096),
                               [(f32_to_bf16_bits(a), runtime.BF16), (f32_to_bf16_bits(a.T.copy()), runtime.BF16)]),
        }
        # one decoder layer (the workload's config 5 sizes) from its StableHLO
        xl, wl, cos, sin = synthetic.decoder_layer_case(rng, 4, 2048, 2048, 16, 128, 8192)
        cases["decoder_layer_B4_S2048"] = (
            programs.decoder_layer(4, 2048, 2048, 16, 128, 8192),
            [(arr, runtime.BF16 if is_bf16 else None)
             for arr, is_bf16 in synthetic.decoder_layer_arguments(xl, wl, cos, sin)])
        # the workload's whole forward (4 layers) as one jitted function
        xs, wss, cos, sin = synthetic.decoder_stack_case(rng, 4, 4, 2048, 2048, 16, 128, 8192)
        cases["decoder_stack_4x_B4_S2048"] = (
            programs.decoder_stack(4, 4, 2048, 2048, 16, 128, 8192),
            [(arr, runtime.BF16 if is_bf16 else None)
             for arr, is_bf16 in synthetic.decoder_stack_arguments(xs, wss, cos, sin)])
        for name, (text, arrays) in cases.items():
            t0 = time.perf_counter()
            exe = client.compile(text)
            compile_ms = (time.perf_counter() - t0) * 1e3
            bufs = [client.buffer(arr, t) if t else client.buffer(arr) for arr, t in arrays]
            times = []
            for i in range(warmup + iters):
                t0 = time.perf_counter()
                outs, done = exe.execute(bufs)
                done.wait()
                dt = time.perf_counter() - t0
                for o in outs:
                    o.close()
                if i == 0:
                    first_ms = dt * 1e3
                if i >= warmup:
                    times.append(dt)
            times.sort()
            out[name] = {"compile_ms": round(compile_ms, 3), "first_call_ms": round(first_ms, 3),
                         "steps": exe.num_steps,
                         "median_us": round(times[len(times) // 2] * 1e6, 2), "min_us": round(times[0] * 1e6, 2),
                         "p90_us": round(times[int(0.9 * (len(times) - 1))] * 1e6, 2), "iters": iters,
                         "warmup": warmup}
            for b in bufs:
                b.close()
            exe.close()
    finally:
        client.close()
    out["int4_g64_M16_K4096_N14336"].update(_c_side_timing(x, packed, s, z, warmup, iters))
    return out


def _c_side_timing(x, packed, s, z, warmup, iters):
    """The int4 headline call timed from C, without Python in the loop: the
    PJRT table as a C caller (jaxlib) drives it, and the host floor under it
    (the kernel library's C-ABI launch plus an event polled to completion),
    both by the harness jax-metallib_amd/lib/test/pjrt_harness."""
    import subprocess
    import tempfile

    lib = os.path.join(REPO, "jax-metallib_amd", "lib")
    harness = os.path.join(lib, "test", "pjrt_harness")
    if not os.path.exists(harness):
        return {"c_side": "pjrt_harness not built"}
    from mi355x import programs

    res = {}
    with tempfile.TemporaryDirectory() as d:
        specs = []
        for name, arr, ptype in (("x", x, 13), ("w", packed, 6), ("s", s, 13), ("z", z, 6)):
            path = os.path.join(d, name + ".bin")
            with open(path, "wb") as f:
                f.write(np.ascontiguousarray(arr).tobytes())
            specs.append(f"{ptype}:{'x'.join(str(v) for v in arr.shape)}:{path}")
        prog = os.path.join(d, "int4.mlir")
        with open(prog, "w") as f:
            f.write(programs.int4_g64_matmul(16, 4096, 14336))
        runs = {"c_table": ["time", os.path.join(lib, "libmk_pjrt.so"), prog, str(warmup), str(iters)] + specs,
                "hip_floor": ["floor", os.path.join(lib, "libmk_kernels.so"), "/opt/rocm/lib/libamdhip64.so",
                              str(warmup), str(iters)]}
        for key, args in runs.items():
            r = subprocess.run([harness] + args, capture_output=True, text=True, timeout=120)
            if r.returncode != 0:
                raise SystemExit(f"bench.py: pjrt_harness {args[0]} failed ({r.returncode}): {r.stderr[-2000:]}")
            res[key] = json.loads(r.stdout.strip().splitlines()[-1])
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--cpu-row-seconds", type=float, default=2.5,
                    help="CPU seconds per secondary line's cpu_baseline (row ops, chain, plumbing)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="",
                    help="comma list of secondary workloads (int8,qmm_m,shard,gemm,decoder,softmax,rmsnorm,argmax,chain6,e2e), "
                         "or 'none'")
    ap.add_argument("--profile", default="",
                    help="comma list of workloads (" + ", ".join(PROFILE_KINDS) + "): eager launches of each in turn "
                         "plus a 256 MiB copy calibration, for rocprofv3 --pmc runs (prints us/launch); layer: the "
                         "decoder layer's "
                         "StableHLO compiled once and executed --steps times (median wall time per call)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one MI355X only (asked for --gpus {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    import torch

    from mi355x import ops

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.profile:
        if args.profile == "layer":
            t = {"layer": profile_layer(args.steps)}
        else:
            t = profile_run(torch, ops, args.profile.split(","), args.steps)
        print(json.dumps({"profile": args.profile, "us_per_launch": {k: round(v * 1e6, 3) for k, v in t.items()},
                          "steps": args.steps}), flush=True)
        return
    only = set(filter(None, args.only.split(",")))

    log(f"[bench] int4 g64 M=16 K=4096 N=14336: steps={args.steps} warmup={args.warmup}")
    r4 = bench_int4(torch, ops, args.steps, args.warmup)
    log(f"[bench] int4: {r4['sec_per_call'] * 1e6:.2f} us/call, {r4['gbs']:.1f} GB/s")
    secondary = {}
    if not only or "int8" in only:
        r8 = bench_int8(torch, ops, args.steps, args.warmup)
        log(f"[bench] int8: {r8['sec_per_call'] * 1e6:.2f} us/call, {r8['gbs']:.1f} GB/s")
        int8_traffic, int8_note = traffic_from_profiles("int8pc_wide_kernel_M16_K4096_N14336")
        secondary["int8_pc_dequant_matmul_M16"] = {
            "value": round(r8["gbs"], 2), "unit": "GB/s", "us_per_call": round(r8["sec_per_call"] * 1e6, 3),
            "roofline": {"bound": "hbm", "achieved": round(r8["gbs"], 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r8["gbs"] / HBM_PEAK_GBS, 4), "traffic": int8_traffic,
                         "traffic_note": int8_note},
        }
        if not args.no_cpu:
            secondary["int8_pc_dequant_matmul_M16"]["cpu_baseline"] = cpu_baseline_qmm("int8", args.cpu_row_seconds)

    def want(name):
        return not only or name in only

    if want("qmm_m"):
        # The rest of the workload's quantized sweep (M in {1, 16, 256, 4096}).
        for M in (1, 256, 4096):
            steps_m = args.steps if M == 1 else max(20, args.steps // (20 if M == 256 else 100))
            for fmt, fn in (("int4", bench_int4), ("int8", bench_int8)):
                r = fn(torch, ops, steps_m, 5, M=M)
                tf = 2 * M * 4096 * 14336 / r["sec_per_call"] / 1e12
                log(f"[bench] {fmt} M={M}: {r['sec_per_call'] * 1e6:.1f} us, {r['gbs']:.0f} GB/s, {tf:.1f} TFLOP/s")
                if M == 1:
                    entry = _hbm_entry(r["gbs"], r["sec_per_call"] * 1e6, {"tflops": round(tf, 2)},
                                       profile=f"{'int4g64' if fmt == 'int4' else 'int8pc'}_M1_K4096_N14336")
                else:
                    entry = {"value": round(tf, 2), "unit": "TFLOP/s", "us_per_call": round(r["sec_per_call"] * 1e6, 3),
                             "gbs": round(r["gbs"], 2),
                             "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS,
                                          "unit": "TFLOP/s", "frac": round(tf / BF16_PEAK_TFLOPS, 4),
                                          "traffic": None}}
                    if M == 256:
                        qt, qn = traffic_from_profiles(
                            "qgemm_ws_kernel_M256_K4096_N14336" if fmt == "int4"
                            else "qgemm_ws_kernel_int8_M256_K4096_N14336")
                        entry["roofline"].update({"traffic": qt, "traffic_note": qn})
                    if M == 4096:
                        # The route's GEMM (the MFMA roofline above; same
                        # kernel and shape for both formats) and its
                        # HBM-bound first pass (W -> bf16) beside it.
                        gt, gn = traffic_from_profiles("gemm_bf16_256dma_kernel_4096x14336x4096")
                        entry["roofline"].update({"traffic": gt, "traffic_note": gn})
                        dt, dn = traffic_from_profiles(f"qmm_dequant_kernel_{fmt}_K4096_N14336")
                        entry["dequant_pass"] = {
                            "kernel": f"qmm_dequant_kernel<{'true' if fmt == 'int4' else 'false'}>",
                            "algorithmic_bytes": 149553152 if fmt == "int4" else 176218112,
                            "traffic": dt, "traffic_note": dn}
                if not args.no_cpu:
                    entry["cpu_baseline"] = cpu_baseline_qmm(fmt, args.cpu_row_seconds, M=M,
                                                             unit="GB/s" if M == 1 else "TFLOP/s")
                secondary[f"{fmt}_dequant_matmul_M{M}"] = entry

    if want("shard"):
        # One GPU's share when the quantized matmul shards by N over 8 GPUs
        # (N = 14336 / 8 = 1792 per GPU, no exchange): the per-shard kernel
        # at its real shape.
        for fmt, fn in (("int4", bench_int4), ("int8", bench_int8)):
            r = fn(torch, ops, args.steps, 5, M=16, K=4096, N=1792)
            log(f"[bench] {fmt} per-shard M=16 N=1792: {r['sec_per_call'] * 1e6:.2f} us, {r['gbs']:.0f} GB/s")
            secondary[f"{fmt}_dequant_matmul_M16_shard_N1792"] = _hbm_entry(
                r["gbs"], r["sec_per_call"] * 1e6,
                {"what": "one of 8 GPUs' share of the headline shape when sharded by N (K=4096, N=1792)"},
                profile=f"{'int4g64' if fmt == 'int4' else 'int8pc'}_shard_M16_K4096_N1792")
            if not args.no_cpu:
                secondary[f"{fmt}_dequant_matmul_M16_shard_N1792"]["cpu_baseline"] = cpu_baseline_qmm(
                    fmt, args.cpu_row_seconds, M=16, N=1792)

    if want("gemm"):
        log("[bench] bf16 GEMM 4096^3 ...")
        rg = bench_gemm_bf16(torch, ops, max(50, args.steps // 20), 5)
        log(f"[bench] bf16 gemm: {rg['sec_per_call'] * 1e6:.1f} us, {rg['tflops']:.1f} TFLOP/s")
        try:
            ref_tf = round(bench_torch_matmul(torch, max(50, args.steps // 20), 5), 2)
            log(f"[bench] torch.matmul (hipBLASLt) 4096^3: {ref_tf} TFLOP/s")
        except Exception as e:  # the comparison is context only
            ref_tf = None
            log(f"[bench] torch.matmul comparison failed: {e}")
        gemm_traffic, gemm_note = traffic_from_profiles("gemm_bf16_256dma_kernel_4096")
        cpu_gemm = None
        if not args.no_cpu:
            cpu_gemm = cpu_baseline_gemm(args.cpu_seconds)
            log(f"[bench] cpu gemm: {cpu_gemm['value']} TFLOP/s on {cpu_gemm['cores']} cores")
        secondary["bf16_gemm_4096"] = {
            "value": round(rg["tflops"], 2), "unit": "TFLOP/s", "us_per_call": round(rg["sec_per_call"] * 1e6, 3),
            "vendor_library_tflops": ref_tf,
            "roofline": {"bound": "mfma", "achieved": round(rg["tflops"], 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(rg["tflops"] / BF16_PEAK_TFLOPS, 4),
                         "traffic": gemm_traffic, "traffic_note": gemm_note},
            "cpu_baseline": cpu_gemm}
        rb = bench_gemm_bf16(torch, ops, max(50, args.steps // 20), 5, batch=16, M=2048, N=2048, K=128)
        gbs = rb["bytes"] / rb["sec_per_call"] / 1e9
        log(f"[bench] batched bf16 gemm: {rb['sec_per_call'] * 1e6:.1f} us, {rb['tflops']:.1f} TFLOP/s, {gbs:.0f} GB/s")
        secondary["bf16_bmm_16x2048x128x2048"] = _hbm_entry(gbs, rb["sec_per_call"] * 1e6,
                                                           {"tflops": round(rb["tflops"], 2)},
                                                           profile="gemm_bf16_batched_16x2048x128x2048")
        if not args.no_cpu:
            secondary["bf16_bmm_16x2048x128x2048"]["cpu_baseline"] = cpu_baseline_bmm(args.cpu_row_seconds)
        rf = bench_gemm_f32(torch, ops, max(50, args.steps // 20), 5)
        log(f"[bench] f32 gemm 2048^3: {rf['sec_per_call'] * 1e6:.1f} us, {rf['tflops']:.1f} TFLOP/s")
        ft, fnote = traffic_from_profiles("gemm_f32_kernel_2048")
        secondary["f32_gemm_2048"] = {
            "value": round(rf["tflops"], 2), "unit": "TFLOP/s", "us_per_call": round(rf["sec_per_call"] * 1e6, 3),
            "roofline": {"bound": "mfma", "achieved": round(rf["tflops"], 2), "peak": 157.3,
                         "unit": "TFLOP/s", "frac": round(rf["tflops"] / 157.3, 4), "traffic": ft,
                         "traffic_note": fnote}}
        if not args.no_cpu:
            secondary["f32_gemm_2048"]["cpu_baseline"] = cpu_baseline_gemm_f32(args.cpu_row_seconds)
    if want("decoder"):
        rd = bench_decoder(torch)
        log(f"[bench] decoder forward: {rd['ms']:.3f} ms, {rd['tokens_per_s']:.0f} tokens/s, {rd['tflops']:.1f} TFLOP/s")
        secondary["llama_decoder_forward_4x2048_b4s2048_int4"] = {
            "value": round(rd["tokens_per_s"], 1), "unit": "tokens/s", "ms_per_forward": round(rd["ms"], 4),
            "roofline": {"bound": "mfma", "achieved": round(rd["tflops"], 2), "peak": BF16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(rd["tflops"] / BF16_PEAK_TFLOPS, 4), "traffic": None},
            "config": rd["config"]}
        if not args.no_cpu:
            cpu_dec = cpu_baseline_decoder()
            log(f"[bench] cpu decoder: {cpu_dec['value']} tokens/s")
            secondary["llama_decoder_forward_4x2048_b4s2048_int4"]["cpu_baseline"] = cpu_dec
    for kind in ("softmax", "rmsnorm", "argmax", "chain6"):
        if not want(kind):
            continue
        for dt in ("f32", "bf16"):
            r = bench_rowop(torch, ops, kind, dt, max(50, args.steps // 10), 5)
            log(f"[bench] {kind} {dt} 8192x8192: {r['sec_per_call'] * 1e6:.1f} us, {r['gbs']:.0f} GB/s")
            prof = (f"mk_ew_jit_chain6_{dt}_8192x8192" if kind == "chain6"
                    else f"row_wave_kernel_{kind}_{dt}_8192x8192" if (kind, dt) == ("argmax", "bf16")
                    else f"row_cached_kernel_{kind}_{dt}_8192x8192")
            entry = _hbm_entry(r["gbs"], r["sec_per_call"] * 1e6, profile=prof)
            if not args.no_cpu:
                entry["cpu_baseline"] = cpu_baseline_rowop(kind, dt, args.cpu_row_seconds)
                log(f"[bench] cpu {kind} {dt}: {entry['cpu_baseline']['value']} GB/s")
            secondary[f"{kind}_{dt}_8192x8192"] = entry

    if want("e2e"):
        e2e = bench_end_to_end()
        for k, v in e2e.items():
            log(f"[bench] end to end {k}: compile {v['compile_ms']} ms, first call {v['first_call_ms']} ms, "
                f"median {v['median_us']} us per execute + await")
        if not args.no_cpu and "plumbing_tanh_matmul_sum_1024" in e2e:
            e2e["plumbing_tanh_matmul_sum_1024"]["cpu_baseline"] = cpu_baseline_plumbing(args.cpu_row_seconds)
            log(f"[bench] cpu plumbing: {e2e['plumbing_tanh_matmul_sum_1024']['cpu_baseline']['value']} us/call")
        secondary["plugin_end_to_end"] = {
            "what": "mkrt_compile once, then mkrt_execute + event await per call, inputs resident; "
                    "wall clock on the host, not kernel time", **e2e}
        st = e2e.get("decoder_stack_4x_B4_S2048")
        if st:
            from mi355x import decoder
            cfg = decoder.DecoderConfig()
            ms = st["median_us"] / 1e3
            tf = cfg.matmul_flops() / ms / 1e9
            log(f"[bench] decoder forward through jit (compile -> execute): {ms:.3f} ms, "
                f"{cfg.tokens / ms * 1e3:.0f} tokens/s, {tf:.1f} TFLOP/s")
            secondary["llama_decoder_forward_jit_4x2048_b4s2048_int4"] = {
                "what": "the 4-layer forward's StableHLO (mi355x/programs.decoder_stack) compiled once by the "
                        "plugin runtime, median of execute + await (host wall clock)",
                "value": round(cfg.tokens / ms * 1e3, 1), "unit": "tokens/s", "ms_per_forward": round(ms, 4),
                "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                             "frac": round(tf / BF16_PEAK_TFLOPS, 4), "traffic": None},
                "plan_steps": st["steps"]}
            if not args.no_cpu:
                # The same workload as the hand-fused line: its CPU figure.
                hand = secondary.get("llama_decoder_forward_4x2048_b4s2048_int4", {})
                secondary["llama_decoder_forward_jit_4x2048_b4s2048_int4"]["cpu_baseline"] = (
                    hand.get("cpu_baseline") or cpu_baseline_decoder())

    cpu = None
    if not args.no_cpu:
        log("[bench] cpu baseline (oracle C port) ...")
        cpu = cpu_baseline_int4(args.cpu_seconds)
        log(f"[bench] cpu: {cpu['value']} GB/s on {cpu['cores']} cores")

    gbs = r4["gbs"]
    int4_traffic, int4_note = traffic_from_profiles("int4g64_wide_kernel_M16_K4096_N14336")
    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r4["sec_per_call"] * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "int4 g64 dequant-matmul, x bf16 [16,4096] @ W uint4 [4096,14336] "
                               "(packed [2048,14336] u8, bf16 scale + u8 zero per 64 k), bf16 out",
                   "M": 16, "K": 4096, "N": 14336, "input_sets": r4["nsets"]},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": int4_traffic,
                     "traffic_note": int4_note},
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
