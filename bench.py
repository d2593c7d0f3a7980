"""Benchmark of the quantized-weight matmul path on one MI355X.

Headline (value): matmulQ4 decode GEMV, M=1, Smith weight [K=4096, N=4096]
quantized with quantizeQ4 (benchmark configuration 1), weights resident in HBM.
A step = one matmulQ4 call (one fused MFMA GEMV launch).  The timed steps
rotate over >= 400 MB of distinct weight copies so the 256 MB MALL cannot
serve them; one rotation of steps is captured as a HIP graph and replayed,
so the time per step is the device's (host launch cost out of the loop);
the same steps launched one by one from Python are reported beside it.
value = algorithmic bytes per step / time per step (GB/s); with one kernel
per step, roofline.achieved is the same figure (a kernel trace of the same
launches averages within ~3 % of it).  headline_q4_0 repeats the measurement
on GGUF Q4_0 blocks (the GGUF decode layout).

Also measured in the same run (under "configs"): Q8 GEMV [4096 x 14336]
(config 2), the Q4 batched-decode sweep (config 3, on quantizeQ4 records and
on GGUF Q4_0 blocks), the Q4 prefill shapes (config 4), the end-to-end
config-5 decode, and the CPU baselines: the oracle's dequantize + f32 matmul
(single thread) on a bounded sample of config 1.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--quick]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
ROTATE_BYTES = 400 << 20
# HBM bytes per config-1 GEMV launch from two rocprofv3 --pmc passes over
# this kernel (FETCH_SIZE, then WRITE_SIZE, per dispatch), FETCH_SIZE scaled
# by the factor a plain device copy of known size gives; the profile named in
# TRAFFIC_SOURCE holds the commands and the figures.
TRAFFIC_CFG1 = 12771509
TRAFFIC_CFG1_Q40 = 9626116
TRAFFIC_SOURCE = "profiles/qgemv1_q4s_m1_cfg1_hbm_traffic.md"
# kernel trace (rocprofv3 --kernel-trace --stats) of the config-1 launches
KERNEL_TRACE = "profiles/qgemv1_cfg1_kernel_trace.md"
KERNEL_CFG1 = "smith_qgemv1_q4s_m1_k128_pl"
KERNEL_CFG1_Q40 = "smith_qgemv1_q40t_m1_k128_pl"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def q4s_bytes(K, N):
    return (K + 31) // 32 * N * 24


def q8_bytes(K, N):
    return (K + 31) // 32 * N * 34


def q40_bytes(K, N):
    return K // 32 * N * 18


def alg_bytes(wbytes, M, K, N):
    return wbytes + 4 * M * K + 4 * M * N


class Weights:
    """R device copies of one quantized weight (R chosen to exceed the MALL)."""

    def __init__(self, D, buf, nbytes, extra=None):
        self.nbytes = nbytes
        reps = max(2, -(-ROTATE_BYTES // nbytes))
        self.bufs = [buf]
        self.extra = [extra] if extra is not None else None
        for _ in range(reps - 1):
            b = D.alloc(nbytes)
            D.check(D.lib.smith_copy_d2d(D.ops_ctx(), b, 0, buf, 0, nbytes))
            self.bufs.append(b)
            if extra is not None:
                eb = D.alloc(extra[1])
                D.check(D.lib.smith_copy_d2d(D.ops_ctx(), eb, 0, extra[0], 0, extra[1]))
                self.extra.append((eb, extra[1]))
        D.sync()


def time_steps(D, step, steps, warmup, rotation=1, graph=False, probe=()):
    """ms per step over exactly `steps` calls, HIP events on the library
    stream around the timed region, and the number of kernel launches one
    step makes (counted in a separate, untimed pass).  graph=True: the
    `steps` calls (step i on weight copy i % rotation, each its own launches)
    are captured once as a HIP graph, replayed once untimed, then replayed
    once timed (launch-bound loops go through graphs).  SMITH_BENCH_EAGER=1
    runs every step eagerly instead (kernel traces: the tracer sees each
    launch)."""
    if os.environ.get("SMITH_BENCH_EAGER") == "1":
        graph = False
    for i in range(warmup):
        step(i)
    D.sync()
    g = None
    if graph:
        D.check(D.lib.smith_graph_begin(D.ops_ctx()), "graph begin")
        try:
            for i in range(steps):
                step(i)
        finally:
            g = D.lib.smith_graph_end(D.ops_ctx())
        if not g:
            D.check(-1, "graph end")
        D.check(D.lib.smith_graph_launch(D.ops_ctx(), g), "graph launch")  # warm
        D.sync()
    D.timer_start()
    if g is not None:
        D.check(D.lib.smith_graph_launch(D.ops_ctx(), g), "graph launch")
    else:
        for i in range(steps):
            step(i)
    ms = D.timer_stop()
    if g is not None:
        D.lib.smith_graph_destroy(g)
    D.profile_kernels(True)
    step(0)
    # which of the `probe` kernel names (longest first: prefixes) one step launched
    kernel, launches = None, 0
    for name in probe:
        _, k = D.profile_read(name)
        if k:
            kernel = kernel or name
            launches += k
    _, rest = D.profile_read("")
    launches += rest
    D.profile_kernels(False)
    return ms / steps, {"launches_per_step": launches, "steps_timed": steps, "graph": g is not None,
                        "kernel": kernel}


_Q4S_CACHE = {}


def q4s_weights(D, S, prng, K, N):
    if (K, N) not in _Q4S_CACHE:
        q = S.quantizeQ4(prng.randn((K, N), 1, std=0.02))
        _Q4S_CACHE[(K, N)] = Weights(D, q["buffer"], q["totalBytes"])
    return _Q4S_CACHE[(K, N)]


def bench_q4s(D, S, prng, M, K, N, steps, warmup, graph=False, probe=()):
    W = q4s_weights(D, S, prng, K, N)
    a = S.tensor(prng.randn((M, K), 0))
    out = S.create([M, N])
    ctx = D.ops_ctx()
    G = (K + 31) // 32
    bufs = W.bufs

    def step(i):
        D.lib.smith_matmul_q4(ctx, a.buffer, bufs[i % len(bufs)], out.buffer, M, N, K, G)

    ms, kt = time_steps(D, step, steps, warmup, rotation=len(bufs), graph=graph, probe=probe)
    return ms, kt, alg_bytes(q4s_bytes(K, N), M, K, N)


def bench_q8(D, S, prng, M, K, N, steps, warmup, graph=False):
    q = S.quantizeQ8(prng.randn((K, N), 1, std=0.02))
    W = Weights(D, q["buffer"], q["totalBytes"])
    a = S.tensor(prng.randn((M, K), 0))
    out = S.create([M, N])
    ctx = D.ops_ctx()
    G = (K + 31) // 32
    bufs = W.bufs

    def step(i):
        D.lib.smith_matmul_q8(ctx, a.buffer, bufs[i % len(bufs)], out.buffer, M, N, K, G)

    ms, kt = time_steps(D, step, steps, warmup, graph=graph)
    for b in bufs[1:]:
        D.release_buffer(b)
    return ms, kt, alg_bytes(q8_bytes(K, N), M, K, N)


def bench_q40(D, S, prng, M, K, N, steps, warmup, graph=False, probe=()):
    """GGUF Q4_0 blocks as the GGUF decode path holds them: nibble and scale
    planes in 16-column tile-major order (smith_repack_q4_0_t_into), through
    smith_linear_q4_0_t (the same GEMV kernels as matmulQ4 for M <= 32)."""
    ctx = D.ops_ctx()
    x = S.tensor(prng.randn((N, K), 1, std=0.02))  # GGUF listing [out, in]
    G = K // 32
    blocks = D.alloc(N * G * 18)
    D.check(D.lib.smith_quantize_q4_0(ctx, x.buffer, blocks, N, K))
    nib = D.alloc(N * G * 16)
    dsc = D.alloc(N * G * 2)
    D.check(D.lib.smith_repack_q4_0_t_into(ctx, blocks, nib, dsc, N, K, 0, 1, N))
    W = Weights(D, nib, N * G * 16, extra=(dsc, N * G * 2))
    a = S.tensor(prng.randn((M, K), 0))
    out = S.create([M, N])

    def step(i):
        j = i % len(W.bufs)
        D.lib.smith_linear_q4_0_t(ctx, a.buffer, W.bufs[j], W.extra[j][0], out.buffer, M, N, K, None, 0.0, None, 0)

    ms, kt = time_steps(D, step, steps, warmup, rotation=len(W.bufs), graph=graph, probe=probe)
    for b in W.bufs[1:]:
        D.release_buffer(b)
    for eb, _ in W.extra[1:]:
        D.release_buffer(eb)
    for b in (blocks, nib, dsc):
        D.release_buffer(b)
    return ms, kt, alg_bytes(q40_bytes(K, N), M, K, N)


def bench_cfg4(D, S, prng, steps=5):
    """Config 4: matmulQ4 at M in {512, 2048} on the MFMA GEMM path.  TFLOP/s
    per step (activation prep + GEMM [+ K-split reduce]) and of the GEMM
    kernel alone (per-launch HIP events of the smith_gemm_q4s_* launches)."""
    pre = {}
    for (Nn, Kk) in [(14336, 4096), (4096, 14336)]:
        for M in (512, 2048):
            msx, ktx, bx = bench_q4s(D, S, prng, M, Kk, Nn, steps, 1)
            fl = 2.0 * M * Nn * Kk
            W = q4s_weights(D, S, prng, Kk, Nn)
            a = S.tensor(prng.randn((M, Kk), 0))
            out = S.create([M, Nn])
            D.profile_kernels(True)
            for i in range(steps):
                D.lib.smith_matmul_q4(D.ops_ctx(), a.buffer, W.bufs[i % len(W.bufs)], out.buffer, M, Nn, Kk,
                                      (Kk + 31) // 32)
            kms, kn = D.profile_read("smith_gemm_q4s")
            kms2, kn2 = D.profile_read("smith_gemm2_q4s")  # the DMA-staged kernels
            kms, kn = kms + kms2, kn + kn2
            D.profile_read("")  # drop the other records (activation prep, reduce)
            D.profile_kernels(False)
            kus = kms * 1e3 / max(kn, 1)
            pre["M%d_N%d_K%d" % (M, Nn, Kk)] = {
                "TFLOPs_step": round(fl / msx / 1e9, 2),
                "mfma_util_vs_f16_dense": round(fl / msx / 1e9 / MFMA_F16_PEAK_TFLOPS, 4),
                "ms_step": round(msx, 3), "kernels_per_step": ktx["launches_per_step"],
                "gemm_kernel_us": round(kus, 1), "gemm_kernel_TFLOPs": round(fl / kus / 1e6, 1),
                "gemm_kernel_mfma_util": round(fl / kus / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
                "path": "f16 activation prep + MFMA GEMM (Q4S dequantized to f16 in LDS, f32 accumulation)"}
            log("cfg4 M=%d N=%d K=%d:" % (M, Nn, Kk), pre["M%d_N%d_K%d" % (M, Nn, Kk)])
    return pre


def bench_cfg4_library_f16():
    """Reference point for config 4: the vendor library's plain f16 GEMM
    (torch.matmul -> hipBLASLt) on already-dequantized f16 weights of the same
    shapes -- no quantized weights, no dequantization, f16 activations.  Not
    part of the product path; it shows the MFMA utilisation a tuned library
    reaches on these shapes.  Run in a child process: torch's wheel carries
    its own HIP runtime, which does not initialise in a process where this
    build's library already holds the GPU."""
    import subprocess
    r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cfg4-library-child"], capture_output=True,
                       text=True, timeout=300)
    if r.returncode != 0:
        return {"error": r.stderr.strip().splitlines()[-1] if r.stderr.strip() else "rc %d" % r.returncode}
    return json.loads(r.stdout.strip().splitlines()[-1])


def _cfg4_library_child(steps=50):
    import torch
    out = {}
    for (Nn, Kk) in [(14336, 4096), (4096, 14336)]:
        for M in (512, 2048):
            a = torch.randn(M, Kk, device="cuda", dtype=torch.float16)
            ws = [torch.randn(Kk, Nn, device="cuda", dtype=torch.float16) for _ in range(4)]
            for i in range(10):
                torch.matmul(a, ws[i % 4])
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for i in range(steps):
                torch.matmul(a, ws[i % 4])
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / steps
            fl = 2.0 * M * Nn * Kk
            out["M%d_N%d_K%d" % (M, Nn, Kk)] = {"us": round(us, 1), "TFLOPs": round(fl / us / 1e6, 1),
                                                "mfma_util_vs_f16_dense": round(fl / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4)}
            del a, ws
    return out


def cpu_baseline(K, N, budget_s):
    """Oracle dequantize + f32 matmul (the reference's CPU semantics), 1 thread."""
    from oracle import oracle as O
    from smith_amd import prng
    w = prng.randn((K, N), 1, std=0.02)
    a = prng.randn((1, K), 0)
    q = O.quantize_q4s(w)
    wd = np.empty((K, N), np.float32)  # reused: the timed loop pays no page faults
    reps, t0 = 0, time.perf_counter()
    while True:
        O.matmul_f32(a, O.dequant_q4s(q, K, N, wd))
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and reps >= 2:
            break
    per = el / reps
    return {"value": round(alg_bytes(q4s_bytes(K, N), 1, K, N) / per / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": "%d x [oracle_dequant_q4s + oracle_matmul_f32] on config 1 (M=1, K=N=4096), %.1f s, "
                      "%.1f ms/call; host has %d cpus" % (reps, el, per * 1e3, os.cpu_count() or 0)}


def cpu_baseline_q8(K, N, budget_s):
    """Config 2 on the CPU: the oracle's Q8 dequantize + f32 matmul (the
    reference's CPU semantics), 1 thread."""
    from oracle import oracle as O
    from smith_amd import prng
    w = prng.randn((K, N), 1, std=0.02)
    a = prng.randn((1, K), 0)
    q = O.quantize_q8(w)
    del w
    wd = np.empty((K, N), np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        O.matmul_f32(a, O.dequant_q8(q, K, N, wd))
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s and reps >= 2:
            break
    per = el / reps
    return {"value": round(alg_bytes(q8_bytes(K, N), 1, K, N) / per / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": "%d x [oracle_dequant_q8 + oracle_matmul_f32] on config 2 (M=1, K=4096, N=14336), %.1f s, "
                      "%.1f ms/call" % (reps, el, per * 1e3)}


def cpu_baseline_gemm(K, N, rows=8):
    """Config 4 on the CPU: the oracle's Q4S dequantize + f32 matmul of a
    sample of `rows` activation rows (the f32 loop is linear in M, so the
    rate holds for M = 512 / 2048), 1 thread."""
    from oracle import oracle as O
    from smith_amd import prng
    w = prng.randn((K, N), 3, std=0.02)
    q = O.quantize_q4s(w)
    del w
    a = prng.randn((rows, K), 20)
    wd = np.empty((K, N), np.float32)
    wd.fill(0.0)  # pages touched before the timed call
    t0 = time.perf_counter()
    O.matmul_f32(a, O.dequant_q4s(q, K, N, wd))
    el = time.perf_counter() - t0
    return {"value": round(2.0 * rows * K * N / el / 1e12, 6), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": "oracle_dequant_q4s + oracle_matmul_f32 of %d rows of config 4 (K=%d, N=%d) in %.1f s, "
                      "rate taken as the M = 512 / 2048 rate" % (rows, K, N, el)}


def cpu_baseline_e2e(reps=2, pos=192):
    """Config-5 decode on the CPU, the reference's path (weights dequantized
    to f32 at load, gguf_loader.js:236; f32 GEMVs per token), 1 thread: one
    layer timed piece by piece -- the seven projections with the oracle's
    f32 matmul, the two RMSNorms, the whole-row RoPE of q and k, 24 heads
    of attention over `pos` cached keys (the middle of the 128 generated
    tokens), SwiGLU and the residuals (oracle/llama_oracle.py) -- times 32,
    plus the LM head; extrapolated from that one layer."""
    from oracle import llama_oracle as LO
    from oracle import oracle as O
    from smith_amd import prng
    c = dict(dim=3072, kv=1024, ffn=9216, vocab=32000, layers=32, heads=24, kvh=8, hd=128)
    shapes = [(c["dim"], c["dim"]), (c["dim"], c["kv"]), (c["dim"], c["kv"]), (c["dim"], c["dim"]),
              (c["dim"], c["ffn"]), (c["dim"], c["ffn"]), (c["ffn"], c["dim"])]
    t_proj = 0.0
    for i, (K, N) in enumerate(shapes):
        w = prng.randn((K, N), 100 + i, std=0.02)
        a = prng.randn((1, K), 0)
        best = None
        for _ in range(reps):
            t0 = time.perf_counter()
            O.matmul_f32(a, w)
            el = time.perf_counter() - t0
            best = el if best is None else min(best, el)
        t_proj += best
        del w
    # the rest of a layer at position pos, on float64 host vectors
    x = prng.randn((1, c["dim"]), 1).astype(np.float64)
    g = np.ones(c["dim"])
    # whole-row RoPE reads table entry pos * (dim / 2) + i
    cos, sin = LO.precompute_rope(c["hd"], (pos + 1) * c["dim"] // c["hd"] + 1, 10000.0)
    Kc = prng.randn((c["kvh"], pos, c["hd"]), 2).astype(np.float64)
    Vc = prng.randn((c["kvh"], pos, c["hd"]), 3).astype(np.float64)
    q = prng.randn((1, c["dim"]), 4).astype(np.float64)
    k = prng.randn((1, c["kv"]), 5).astype(np.float64)
    gu = prng.randn((2, c["ffn"]), 6).astype(np.float64)
    best = None
    for _ in range(max(reps, 3)):
        t0 = time.perf_counter()
        n1 = LO.rmsnorm(x, g, 1e-5)
        LO.rope_rows(q, pos, cos, sin)
        LO.rope_rows(k, pos, cos, sin)
        att = np.empty(c["dim"])
        for h in range(c["heads"]):
            kv = h // (c["heads"] // c["kvh"])
            att[h * c["hd"]:(h + 1) * c["hd"]] = LO.attend(q[0, h * c["hd"]:(h + 1) * c["hd"]], Kc[kv], Vc[kv],
                                                           1.0 / np.sqrt(c["hd"]))
        x2 = x + n1
        LO.rmsnorm(x2, g, 1e-5)
        h_ = LO.swiglu(gu[0], gu[1])
        x2 + h_[:c["dim"]]
        el = time.perf_counter() - t0
        best = el if best is None else min(best, el)
    t_rest = best
    w = prng.randn((c["dim"], c["vocab"]), 200, std=0.02)
    t0 = time.perf_counter()
    O.matmul_f32(prng.randn((1, c["dim"]), 0), w)
    t_head = time.perf_counter() - t0
    del w
    per_token = c["layers"] * (t_proj + t_rest) + t_head
    return {"value": round(1.0 / per_token, 4), "unit": "tokens/s", "cores": 1, "kind": "port",
            "sample": "one config-5 layer on the CPU: oracle f32 GEMVs of its seven projections (%.1f ms, best of "
                      "%d) + RMSNorms, whole-row RoPE, 24-head attention over %d cached keys, SwiGLU, residuals "
                      "(%.2f ms), x 32 layers, + the LM head (%.1f ms); extrapolated from one layer"
                      % (t_proj * 1e3, reps, pos, t_rest * 1e3, t_head * 1e3)}


_FLOOR_LIB = None


def floor_us(name, bufs, n, out, grid, block, steps):
    """Per-launch us of a bench-only floor kernel (smith_bench.hsaco, through
    libsmith_bench.so): `steps` launches, launch i reading bufs[i % len],
    captured as one HIP graph and replayed (timed like the product's steps)."""
    import ctypes
    global _FLOOR_LIB
    lib_dir = os.path.join(ROOT, "smith_amd", "lib")
    if _FLOOR_LIB is None:
        _FLOOR_LIB = ctypes.CDLL(os.path.join(lib_dir, "libsmith_bench.so"))
        _FLOOR_LIB.smith_bench_floor.restype = ctypes.c_int
        _FLOOR_LIB.smith_bench_floor.argtypes = [
            ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint32, ctypes.c_uint64,
            ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_double)]
        _FLOOR_LIB.smith_bench_error.restype = ctypes.c_char_p
    arr = (ctypes.c_void_p * len(bufs))(*[int(b) for b in bufs])
    us = ctypes.c_double()
    rc = _FLOOR_LIB.smith_bench_floor(os.path.join(lib_dir, "smith_bench.hsaco").encode(), name.encode(), arr,
                                      len(bufs), n, int(out), grid, block, steps, ctypes.byref(us))
    if rc != 0:
        raise RuntimeError("floor kernel %s: %s" % (name, _FLOOR_LIB.smith_bench_error().decode()))
    return us.value


def calibrate(D, steps):
    """Platform floor: per-launch duration of an empty kernel and of a plain
    128-bit streaming read of the config-1/3 weight sizes (graph-replayed
    launches, buffers rotated over >= 800 MB)."""
    res = {}
    out = D.alloc(4096)
    for name in ("floor_empty", "floor_stream_read", "floor_block_read"):
        for size in (12582912, 44040192, 201326592):
            reps = max(2, -(-(800 << 20) // size))
            bufs = [D.alloc(size) for _ in range(reps)]
            for b in bufs:
                D.check(D.lib.smith_fill_zero(D.ctx(), b, size))
            D.sync()
            n16 = size // 16
            grid = (n16 + 767) // 768 if name == "floor_block_read" else 1024
            us = floor_us(name, bufs, n16, out, grid, 128 if name == "floor_block_read" else 256, steps)
            res["%s_%dB" % (name, size)] = {"us": round(us, 2), "GBps": round(size / us / 1e3, 1)}
            for b in bufs:
                D.release_buffer(b)
    return res


def read_floor(D, S, prng, K, N, steps):
    """The config-1 step's floor on this GPU, timed like the headline
    (graph-replayed steps over the same rotated weight copies): an empty
    launch, a plain 16-byte streaming read of the weight bytes, and each
    GEMV's own record loads with its grid and nothing else -- on the Q4S
    records (smith_qgemv1_q4s_m1_k128) and on the GGUF Q4_0 tile planes
    (smith_qgemv1_q40t_m1_k128)."""
    assert K == 4096 and N % 16 == 0
    out = D.alloc(256)
    D.check(D.lib.smith_fill_zero(D.ctx(), out, 256))
    W = q4s_weights(D, S, prng, K, N)
    nb = q4s_bytes(K, N)
    res = {"empty_launch_us": floor_us("floor_empty", W.bufs, nb // 16, out, 1024, 256, steps),
           "stream_read_us": floor_us("floor_block_read", W.bufs, nb // 16, out, (nb // 16 + 767) // 768, 128, steps),
           "q4s_record_read_us": floor_us("floor_q4s_record_read", W.bufs, N, out, N // 16, 512, steps)}
    # Q4_0 tile planes: nibble plane then scale plane in one buffer per copy
    nb40 = q40_bytes(K, N)
    reps = max(2, -(-ROTATE_BYTES // nb40))
    bufs40 = [D.alloc(nb40) for _ in range(reps)]
    for b in bufs40:
        D.check(D.lib.smith_fill_zero(D.ctx(), b, nb40))
    D.sync()
    res["q4_0_stream_read_us"] = floor_us("floor_block_read", bufs40, nb40 // 16, out, (nb40 // 16 + 767) // 768,
                                          128, steps)
    res["q4_0_record_read_us"] = floor_us("floor_q40t_record_read", bufs40, N, out, N // 16, 512, steps)
    for b in bufs40:
        D.release_buffer(b)
    D.sync()
    assert not D.download(out, 256, np.uint8).any()
    D.release_buffer(out)
    return {k: round(v, 3) for k, v in res.items()}


def stream_floor_us(D, nbytes, steps=100):
    """Per-launch us of a plain 16-byte streaming read of `nbytes` (the
    fastest grid shape found, floor_block_read), graph-replayed over copies
    rotated past the MALL: what any kernel reading that many weight bytes
    takes on this GPU, whatever its grid."""
    out = D.alloc(256)
    D.check(D.lib.smith_fill_zero(D.ctx(), out, 256))
    nbytes = -(-nbytes // 16) * 16
    bufs = [D.alloc(nbytes) for _ in range(max(2, -(-ROTATE_BYTES // nbytes)))]
    for b in bufs:
        D.check(D.lib.smith_fill_zero(D.ctx(), b, nbytes))
    D.sync()
    n16 = nbytes // 16
    us = floor_us("floor_block_read", bufs, n16, out, (n16 + 767) // 768, 128, steps)
    D.sync()
    for b in bufs:
        D.release_buffer(b)
    D.release_buffer(out)
    return round(us, 3)


# The decode GEMV variants of configs 1-3: (name suffix, record-read floor
# kernel, threads, grid (N, G) -> (GX, GY)); names longest first (probe
# prefixes), as the bridge names its launches
def _cdiv(a, b):
    return -(-a // b)


GEMV_VARIANTS = [
    ("qgemv1_%s_m1_k448w16_pl", "c1s7w16", 1024, lambda N, G: (_cdiv(N, 16), 1)),
    ("qgemv1_%s_m1_k128_c2", "c2s4w8", 512, lambda N, G: (_cdiv(N, 32), _cdiv(G, 128))),
    ("qgemv1_%s_m1_k128", "c1s4w8", 512, lambda N, G: (_cdiv(N, 16), _cdiv(G, 128))),
    ("qgemv5_%s_m%d_k32c4", "c4s1w8", 512, lambda N, G: (_cdiv(N, 64), _cdiv(G, 32))),
    ("qgemv5_%s_m%d_k64c2", "c2s1w16", 1024, lambda N, G: (_cdiv(N, 32), _cdiv(G, 64))),
    ("qgemv5_%s_m%d_k32", "c1s1w8", 512, lambda N, G: (_cdiv(N, 16), _cdiv(G, 32))),
    ("qgemv5_%s_m%d_w16", "c1s2w16", 1024, lambda N, G: (_cdiv(N, 16), 1)),
]


def gemv_probe(tag, M):
    """Kernel names one config-3 step may launch (prefixes, longest first)."""
    return [_variant_name(fmt, tag, M) for fmt, _, _, _ in GEMV_VARIANTS
            if (M == 1) == fmt.startswith("qgemv1")]


def _bucket(M):
    return 4 if M <= 4 else 8 if M <= 8 else 16 if M <= 16 else 32


def _variant_name(fmt, tag, M):
    return "smith_" + (fmt % tag if fmt.startswith("qgemv1") else fmt % (tag, _bucket(M)))


def record_floor_us(D, bufs, tag, kernel, M, K, N, steps=100):
    """Per-launch us of the launched GEMV's record loads alone (its grid,
    lanes and records; no math, no split-K finish), graph-replayed over the
    rotated zero buffers `bufs`."""
    G = K // 32
    for fmt, suffix, threads, grid in GEMV_VARIANTS:
        if _variant_name(fmt, tag, M) == kernel:
            gx, gy = grid(N, G)
            out = D.alloc(256)
            D.check(D.lib.smith_fill_zero(D.ctx(), out, 256))
            n = N | (G << 20) | (gx << 40)
            us = floor_us("floor_rec_%s_%s" % (tag, suffix), bufs, n, out, gx * gy, threads, steps)
            D.release_buffer(out)
            return round(us, 3)
    raise RuntimeError("no record floor for %s" % kernel)


def _rotated_zeros(D, nbytes):
    nbytes = -(-nbytes // 16) * 16
    bufs = [D.alloc(nbytes) for _ in range(max(2, -(-ROTATE_BYTES // nbytes)))]
    for b in bufs:
        D.check(D.lib.smith_fill_zero(D.ctx(), b, nbytes))
    D.sync()
    return bufs


def _sweep_point(ms, nbytes, launches, floor):
    us = ms * 1e3
    return {"GBps": round(nbytes / ms / 1e6, 1), "pct_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBS * 100, 2),
            "us_step": round(us, 2), "kernels_per_step": launches, "stream_read_us": floor,
            "over_stream_read": round(us / floor, 3) if floor == floor else None}


def bench_sweeps(D, S, prng):
    """Config 2 and the config-3 sweeps (Q4S records and GGUF Q4_0 blocks),
    each point graph-replayed, with the streaming-read floor of its weight
    bytes (stream_read_us; over_stream_read = step / floor) and the
    launched kernel's record loads alone with its grid (record_read_us,
    over_record_read)."""
    eager = os.environ.get("SMITH_BENCH_EAGER") == "1"  # traced runs: no floor graphs
    floor = (lambda nbytes: float("nan")) if eager else (lambda nbytes: stream_floor_us(D, nbytes))
    configs = {}
    sub = 100  # sweep points: enough graph-replayed steps to amortise the graph launch
    ms8, kt8, b8 = bench_q8(D, S, prng, 1, 4096, 14336, sub, 5, graph=True)
    configs["cfg2_q8_gemv_M1_K4096_N14336"] = _sweep_point(ms8, b8, kt8["launches_per_step"],
                                                           floor(q8_bytes(4096, 14336)))
    log("cfg2:", configs["cfg2_q8_gemv_M1_K4096_N14336"])
    for tag, bench_fn, nbytes_fn, key in (("q4s", bench_q4s, q4s_bytes, "cfg3_q4s_batched_decode"),
                                          ("q40t", bench_q40, q40_bytes, "cfg3_q4_0_batched_decode")):
        # (the same sweep on GGUF Q4_0 blocks: 18 B per 32 weights, tile-major planes)
        sweep = {}
        for (Nn, Kk) in [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]:
            fl = floor(nbytes_fn(Kk, Nn))
            # the record floors read zeros laid out as the kernel's weight (Q4_0:
            # nibble plane then scale plane)
            rbufs = None if eager else _rotated_zeros(D, nbytes_fn(Kk, Nn))
            for M in (1, 4, 8, 16, 32):
                msx, ktx, bx = bench_fn(D, S, prng, M, Kk, Nn, sub, 5, graph=True, probe=gemv_probe(tag, M))
                pt = _sweep_point(msx, bx, ktx["launches_per_step"], fl)
                pt["kernel"] = ktx["kernel"]
                if rbufs is not None and ktx["kernel"]:
                    rr = record_floor_us(D, rbufs, tag, ktx["kernel"], M, Kk, Nn)
                    pt["record_read_us"] = rr
                    pt["over_record_read"] = round(msx * 1e3 / rr, 3)
                sweep["M%d_N%d_K%d" % (M, Nn, Kk)] = pt
            for b in rbufs or ():
                D.release_buffer(b)
        configs[key] = sweep
        log(key + ":", json.dumps(sweep))
    return configs


def e2e_weight_bytes(mix):
    """HBM bytes of weights one decode token streams at config 5."""
    c = __import__("smith_amd.synthetic_gguf", fromlist=["CONFIG5"]).CONFIG5
    d, f, v, L = c["dim"], c["ffn"], c["vocab"], c["layers"]
    kv = c["kv_heads"] * d // c["heads"]
    if mix == "q4_0":
        return 1981808640 + 55296000  # Q4_0 linears + Q4_0 LM head
    q4k = L * (2 * d * d + d * kv + 2 * d * f)  # q, o, k, gate, up
    q6k = L * (d * kv + f * d)                  # v, down
    return q4k * 144 // 256 + q6k * 210 // 256 + d * v * 210 // 256  # + the Q6_K LM head


def bench_e2e(D, path, prompt_len=128, new_tokens=128, reps=3, mix="q4_0"):
    """Config 5: seeded synthetic Llama GGUF (Q4_0 linears, or the Q4_K_M
    mix), loadGGUF, then generate(prompt of 128 seeded ids, maxTokens 128,
    temperature 0).  Decode tok/s = decode steps / decode time (HIP events
    around the greedy graph replays); prefill reported separately."""
    from smith_amd import prng
    from smith_amd.gguf_loader import loadGGUF
    from smith_amd.synthetic_gguf import CONFIG5, build_llama_gguf
    t0 = time.perf_counter()
    if not os.path.exists(path):
        c = CONFIG5
        build_llama_gguf(path, dim=c["dim"], layers=c["layers"], heads=c["heads"], kv_heads=c["kv_heads"],
                         ffn=c["ffn"], vocab=c["vocab"], context=c["context"], seed=1, mix=mix)
    t_write = time.perf_counter() - t0
    t0 = time.perf_counter()
    m = loadGGUF(path)
    t_load = time.perf_counter() - t0
    prompt = [int(x) for x in prng.randint(prompt_len, m.config["vocabSize"], 7)]
    m.generate(prompt, {"maxTokens": 4, "temperature": 0})  # warm-up (captures the decode graph)
    best = None
    for _ in range(reps):
        D.timer_start()
        out = m.generate(prompt, {"maxTokens": 1, "temperature": 0})
        t_prefill = D.timer_stop()
        D.timer_start()
        out = m.generate(prompt, {"maxTokens": new_tokens, "temperature": 0})
        t_all = D.timer_stop()
        dec_ms = t_all - t_prefill
        r = {"decode_tok_s": round((new_tokens - 1) / (dec_ms * 1e-3), 1), "decode_ms_per_token": round(dec_ms / (new_tokens - 1), 4),
             "prefill_ms": round(t_prefill, 3), "prefill_tok_s": round(prompt_len / (t_prefill * 1e-3), 1),
             "generate_ms": round(t_all, 3)}
        if best is None or r["decode_tok_s"] > best["decode_tok_s"]:
            best = r
    gb_per_token = e2e_weight_bytes(mix)
    best.update({"mix": mix, "weights_GB_per_token": round(gb_per_token / 1e9, 3),
                 "weight_stream_GBps": round(gb_per_token / (best["decode_ms_per_token"] * 1e-3) / 1e9, 1),
                 "tokens_generated": len(out) - prompt_len, "gguf_write_s": round(t_write, 1),
                 "load_s": round(t_load, 1), "first_tokens": out[prompt_len:prompt_len + 8]})
    # a fast decode of wrong tokens is no measurement: the first tokens must be
    # those of the oracle-checked run (tests/test_gpu_config5.py holds them to
    # the same file)
    with open(os.path.join(ROOT, "tests", "golden", "cfg5_first_tokens.json")) as f:
        want = json.load(f)[mix]
    if best["first_tokens"] != want:
        raise RuntimeError("config 5 (%s): first tokens %s differ from the oracle-checked %s"
                           % (mix, best["first_tokens"], want))
    best["first_tokens_match_fixture"] = True
    return best


def counter_set(D, S, prng, gguf, steps=3):
    """Eager launches for rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE per
    dispatch): a 8 MiB device copy (the scale of FETCH_SIZE), config 1 (Q4S
    and Q4_0 tile planes), config 2, the config-3 sweep on both formats, and
    a config-5 prompt + 8 greedy tokens with every decode step launched
    eagerly (SMITH_DECODE_GRAPH=0).  Each point runs `steps` launches on
    distinct weight copies."""
    src, dst = D.alloc(8 << 20), D.alloc(8 << 20)
    for _ in range(steps):
        D.check(D.lib.smith_copy_d2d(D.ops_ctx(), dst, 0, src, 0, 8 << 20))
    D.sync()
    for b in (src, dst):
        D.release_buffer(b)
    bench_q4s(D, S, prng, 1, 4096, 4096, steps, 1)
    bench_q40(D, S, prng, 1, 4096, 4096, steps, 1)
    bench_q8(D, S, prng, 1, 4096, 14336, steps, 1)
    for (Nn, Kk) in [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]:
        for M in (1, 4, 8, 16, 32):
            bench_q4s(D, S, prng, M, Kk, Nn, steps, 1)
            bench_q40(D, S, prng, M, Kk, Nn, steps, 1)
    from smith_amd.gguf_loader import loadGGUF
    from smith_amd.synthetic_gguf import CONFIG5, build_llama_gguf
    for mix in ("q4_0", "q4_k_m"):
        path = gguf if mix == "q4_0" else gguf.replace(".gguf", "_%s.gguf" % mix)
        if not os.path.exists(path):
            c = CONFIG5
            build_llama_gguf(path, dim=c["dim"], layers=c["layers"], heads=c["heads"], kv_heads=c["kv_heads"],
                             ffn=c["ffn"], vocab=c["vocab"], context=c["context"], seed=1, mix=mix)
        m = loadGGUF(path)
        prompt = [int(x) for x in prng.randint(128, m.config["vocabSize"], 7)]
        out = m.generate(prompt, {"maxTokens": 8, "temperature": 0})
        log("counter set %s: tokens %s" % (mix, out[128:]))
        del m
    D.sync()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--quick", action="store_true", help="headline only, no sweep / cpu baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate", action="store_true", help="print the platform floor (empty kernel, streaming read)")
    ap.add_argument("--e2e-only", action="store_true", help="only the config-5 end-to-end decode")
    ap.add_argument("--cfg4-only", action="store_true", help="only the config-4 prefill GEMMs")
    ap.add_argument("--cfg3-only", action="store_true", help="only the config-2/3 GEMV sweep")
    ap.add_argument("--gguf", default="/tmp/smith_config5.gguf", help="synthetic config-5 GGUF path (written if absent)")
    ap.add_argument("--mix", default="q4_0", choices=["q4_0", "q4_k_m"], help="config-5 weight types for --e2e-only")
    ap.add_argument("--cfg4-library-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--counter-set", action="store_true",
                    help="eager launches of every measured kernel, for rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.counter_set:
        os.environ["SMITH_DECODE_GRAPH"] = "0"  # before smith_amd.gguf_cache is imported
    if args.cfg4_library_child:
        print(json.dumps(_cfg4_library_child()), flush=True)
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (--gpus %d requested); multi-GPU "
              "sharding is not implemented" % args.gpus, file=sys.stderr)
        sys.exit(2)

    import smith_amd as S
    from smith_amd import device as D
    from smith_amd import prng

    D.ops_ctx()
    log("device:", D.device_name())
    if args.counter_set:
        counter_set(D, S, prng, args.gguf)
        return
    if args.calibrate:
        print(json.dumps({"calibration": calibrate(D, args.steps)}), flush=True)
        return
    if args.e2e_only:
        path = args.gguf if args.mix == "q4_0" else args.gguf.replace(".gguf", "_%s.gguf" % args.mix)
        print(json.dumps({"cfg5_e2e": bench_e2e(D, path, mix=args.mix)}), flush=True)
        return
    if args.cfg4_only:
        print(json.dumps({"cfg4_q4s_prefill": bench_cfg4(D, S, prng),
                          "cfg4_library_f16_gemm_reference": bench_cfg4_library_f16()}), flush=True)
        return
    if args.cfg3_only:
        print(json.dumps(bench_sweeps(D, S, prng)), flush=True)
        return
    K = N = 4096
    # The value: matmulQ4 steps captured once as a HIP graph (one launch per
    # step, each step on its own weight copy) and replayed, so the figure is
    # the device's per-step time; the same steps launched one by one from
    # Python (ctypes -> bridge -> hipModuleLaunchKernel, ~4 us of host time
    # per call) are reported beside it
    ms_stream, kt, nbytes = bench_q4s(D, S, prng, 1, K, N, args.steps, args.warmup)
    ms, ktg, _ = bench_q4s(D, S, prng, 1, K, N, args.steps, args.warmup, graph=True)
    assert kt["launches_per_step"] == 1, kt  # the M=1 path is one fused kernel
    value = nbytes / (ms * 1e-3) / 1e9
    # one kernel per step: the timed region's average is that kernel's
    # average launch-to-launch duration on the library stream (a kernel
    # trace of the same launches, eager, averages within ~3 % of it)
    achieved = value
    ms40_stream, kt40, b40 = bench_q40(D, S, prng, 1, K, N, args.steps, args.warmup)
    ms40, _, _ = bench_q40(D, S, prng, 1, K, N, args.steps, args.warmup, graph=True)
    v40 = b40 / (ms40 * 1e-3) / 1e9
    achieved40 = v40
    if os.environ.get("SMITH_BENCH_EAGER") == "1":
        # traced runs: no graph replay at all (the floor kernels only run
        # from a captured graph)
        floor = {k: float("nan") for k in ("empty_launch_us", "stream_read_us", "q4s_record_read_us",
                                           "q4_0_stream_read_us", "q4_0_record_read_us")}
    else:
        floor = read_floor(D, S, prng, K, N, args.steps)
    floor["kernel_over_record_read"] = round(ms * 1e3 / floor["q4s_record_read_us"], 3)
    floor["frac_of_stream_read"] = round(floor["stream_read_us"] / (ms * 1e3), 3)
    floor["q4_0_kernel_over_record_read"] = round(ms40 * 1e3 / floor["q4_0_record_read_us"], 3)
    floor["q4_0_frac_of_stream_read"] = round(floor["q4_0_stream_read_us"] / (ms40 * 1e3), 3)
    log("cfg1 floor:", json.dumps(floor))
    log("cfg1 q4s M=1: %.2f us/step graph = %.0f GB/s, %.2f us/step stream; q4_0: %.2f us graph = %.0f GB/s, %.2f stream"
        % (ms * 1e3, value, ms_stream * 1e3, ms40 * 1e3, v40, ms40_stream * 1e3))

    configs = {}
    if not args.quick:
        configs.update(bench_sweeps(D, S, prng))
        pre = bench_cfg4(D, S, prng)
        configs["cfg4_q4s_prefill"] = pre
        log("cfg4:", json.dumps(pre))
        configs["cfg4_library_f16_gemm_reference"] = bench_cfg4_library_f16()
        log("cfg4 library f16 reference:", json.dumps(configs["cfg4_library_f16_gemm_reference"]))

    cpu = None
    if not args.quick:
        cpu = cpu_baseline(K, N, args.cpu_seconds)
        log("cpu baseline:", cpu)
        configs["cfg2_q8_gemv_M1_K4096_N14336"]["cpu_baseline"] = cpu_baseline_q8(4096, 14336, args.cpu_seconds / 2)
        log("cfg2 cpu baseline:", configs["cfg2_q8_gemv_M1_K4096_N14336"]["cpu_baseline"])
        configs["cfg4_q4s_prefill"]["cpu_baseline"] = cpu_baseline_gemm(4096, 14336)
        log("cfg4 cpu baseline:", configs["cfg4_q4s_prefill"]["cpu_baseline"])
        e2e = bench_e2e(D, args.gguf)
        e2e["cpu_baseline"] = cpu_baseline_e2e()
        e2e["bound_tok_s_at_hbm_peak"] = round(HBM_PEAK_GBS * 1e9 / (1981808640 + 55296000), 1)
        configs["cfg5_e2e_llama_q4_0_decode"] = e2e
        log("cfg5:", json.dumps(e2e))
        km = bench_e2e(D, args.gguf.replace(".gguf", "_q4_k_m.gguf"), mix="q4_k_m", reps=2)
        km["bound_tok_s_at_hbm_peak"] = round(HBM_PEAK_GBS * 1e9 / e2e_weight_bytes("q4_k_m"), 1)
        configs["cfg5_e2e_llama_q4_k_m_decode"] = km
        log("cfg5 q4_k_m:", json.dumps(km))

    line = {
        "metric": "Q4 GEMV GB/s (% HBM peak) + Q4 decode tokens/sec, 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "ms_per_step_stream_launches": round(ms_stream, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 in/out; Q4S weights exact in f16 MFMA operands; activations as f16 hi + lo*2048 pairs "
                 "(~22 bits of each f32 kept) at M<=8, plain f16 at M 9-32; f32 accumulation",
        "data": "synthetic (SplitMix64/Box-Muller seeded: a~N(0,1) seed 0, W~N(0,0.02) seed 1)",
        "config": {"workload": "config 1: matmulQ4 GEMV M=1, Smith weight [K=4096, N=4096] quantizeQ4 (Q4S, "
                               "24 B/32 weights); weights rotated over >= 400 MB of copies",
                   "M": 1, "K": K, "N": N, "format": "Q4S", "algorithmic_bytes_per_step": nbytes,
                   "timing": "HIP events on the library stream around %d steps replayed from a captured HIP graph "
                             "(one kernel launch per step)" % ktg["steps_timed"]},
        "pct_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_CFG1,
                     "traffic_source": TRAFFIC_SOURCE,
                     "kernel": KERNEL_CFG1, "step_us": round(ms * 1e3, 3), "kernel_trace": KERNEL_TRACE},
        "read_floor": dict(floor, target_70pct_q4_0_us=round(b40 / (0.7 * HBM_PEAK_GBS * 1e3), 3),
                           note="same weight bytes and rotation, graph-replayed: empty launch, plain streaming "
                                "read, each GEMV's record loads alone (its grid, no math), for Q4S records and "
                                "Q4_0 tile planes.  The north star's 70 % of HBM peak on config 1 Q4_0 "
                                "(target_70pct_q4_0_us) lies below what a plain streaming read of the same "
                                "bytes takes here (q4_0_stream_read_us), so no kernel reaches it per launch "
                                "at this size"),
        "headline_q4_0": {
            "workload": "config 1 on GGUF Q4_0 blocks (18 B/32 weights, tile-major nibble/scale planes as the "
                        "GGUF loader holds them), smith_linear_q4_0_t M=1, K=N=4096",
            "value": round(v40, 2), "unit": "GB/s", "ms_per_step": round(ms40, 6),
            "ms_per_step_stream_launches": round(ms40_stream, 6), "algorithmic_bytes_per_step": b40,
            "roofline": {"bound": "hbm", "achieved": round(achieved40, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(achieved40 / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_CFG1_Q40,
                         "traffic_source": TRAFFIC_SOURCE, "kernel": KERNEL_CFG1_Q40,
                         "step_us": round(ms40 * 1e3, 3), "kernel_trace": KERNEL_TRACE}},
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
