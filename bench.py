"""Benchmark of golem's quantized linear-layer path on one MI355X.

The headline workload is the benchmark's config 1: the Q6_K output head,
151936 rows x 2560 inputs, batch 1.  One step is one pass of the path over
one token: Q8_K-quantise the activation (Batch.QuantizeK) and run the Q6_K
matrix-vector product (MatVecQ6_K) -- everything resident in HBM before the
timed region.  `value` is algorithmic bytes per step (weights as stored +
quantised activation + fp32 logits) over the step time, in GB/s.

The weights rotate over two resident copies (640 MB together) so that no
step finds the previous step's weights in the 256 MB Infinity Cache.

Also reported, measured the same way with HIP events on the library's
stream: config 0 (Q4_0 matvec 9728x2560, rotating over 20 copies = 281 MB),
config 2 (the Q4_0 x Q8_0 MFMA product at M = 64, 512, 2048) and config 4
(the Gemma-shaped MoE layer: route + experts, decode and a 256-position
prefill).

cpu_baseline: golem's x86 path -- its AVX2 kernels and worker pool, restated
in C with intrinsics (oracle/cpu_avx2.c) -- timed on this host's allowed
threads over a bounded sample of config 1 (and one thread beside it), and
used at the same time to check the GPU's logits bit for bit.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, 5.0 POP/s


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-extra", action="store_true", help="skip the config 0 / config 2 measurements")
    p.add_argument("--only", default="",
                   help="profiling: run only this leg (c1, c0, c0floor, c2, c3, c3prefill, c3eager, c4, valu) and exit; 'copy' runs the 256 MiB "
                        "device copy that scales the FETCH_SIZE / WRITE_SIZE counters; 'c3prefill' reads "
                        "config 3's 512-token prompt four times (a kernel trace of the prefill alone)")
    p.add_argument("--c2-m", type=int, default=0, help="profiling: config 2 at this M only")
    return p.parse_args()


def read_traffic(name):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, scaled by a copy kernel of known size), kept as a one-line
    text summary under profiles/."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1].strip())
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only; --gpus {args.gpus} is not supported by this build "
              "(the products would shard by output rows, one shard a GPU)", file=sys.stderr)
        sys.exit(2)

    import torch
    from golem_amd import capi, synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    torch.cuda.init()
    if args.only == "copy":
        # A plain copy of known size: FETCH_SIZE / WRITE_SIZE per dispatch of
        # it, against 256 MiB read and 256 MiB written, give the factors that
        # turn those counters into bytes.
        n = 256 << 20
        a = torch.full((n // 4,), 1.0, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(5):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"leg": "copy", "bytes": n, "dispatches": 5}))
        return
    stream = torch.cuda.current_stream()
    ctx = capi.Context(0, stream=stream.cuda_stream)
    call = capi.call
    vp = capi.vp

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a).copy()).cuda()

    # ---- config 1: Q6_K head, 151936 x 2560, M = 1, seed 1 ----------------
    rows, cols = 151936, 2560
    g = synth.rng(1)
    w6 = synth.q6_k_weights(g, rows, cols)
    x = synth.activations(g, 1, cols)
    copies = [capi.Weight(ctx, w6, capi.Q6_K, rows, cols) for _ in range(2)]
    xd = dev(x)
    q = torch.empty((1, cols), dtype=torch.int8, device="cuda")
    ks = torch.empty((1, cols // 256), dtype=torch.float32, device="cuda")
    bs = torch.empty((1, cols // 16), dtype=torch.int16, device="cuda")
    y = torch.empty((1, rows), dtype=torch.float32, device="cuda")
    step_bytes = rows * (cols // 256) * 210 + cols + 4 * (cols // 256) + 2 * (cols // 16) + 4 * rows

    def step(i):
        call("gx_quantize_q8_k", ctx.ptr, vp(xd), cols, 1, cols, vp(q), vp(ks), vp(bs))
        call("gx_matmul_q6_k", ctx.ptr, copies[i & 1].ptr, vp(q), vp(ks), vp(bs), 1, 0, rows, None, vp(y), rows)

    if args.only in ("", "c1"):
        for i in range(args.warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms_per_step = (t1 - t0) * 1e3 / args.steps
        value = step_bytes / (ms_per_step * 1e-3) / 1e9

        # The dominant kernel alone, timed with HIP events on the same stream.
        reps = max(args.steps, 50)
        ctx.timer_start()
        for i in range(reps):
            call("gx_matmul_q6_k", ctx.ptr, copies[i & 1].ptr, vp(q), vp(ks), vp(bs), 1, 0, rows, None, vp(y),
                 rows)
        kernel_ms = ctx.timer_stop() / reps
        matvec_bytes = rows * (cols // 256) * 210 + cols + 4 * (cols // 256) + 2 * (cols // 16) + 4 * rows
        achieved = matvec_bytes / (kernel_ms * 1e-3) / 1e9
        if args.only == "c1":
            print(json.dumps({"leg": "c1", "ms_per_step": ms_per_step, "kernel_ms": kernel_ms}))
            return

    # ---- config 0 and config 2 (secondary) --------------------------------
    extra = {}
    if not args.no_extra and args.only in ("", "c0", "c0floor", "c2"):
        r0, c0 = 9728, 2560
        g0 = synth.rng(0)
        w0 = synth.q4_0_weights(g0, r0, c0)
        x0 = synth.activations(g0, 1, c0)
        if args.only in ("", "c0", "c0floor"):
            n_copies = 20
            w0s = [capi.Weight(ctx, w0, capi.Q4_0, r0, c0) for _ in range(n_copies)]
            x0d = dev(x0)
            q0 = torch.empty((1, c0), dtype=torch.int8, device="cuda")
            s0 = torch.empty((1, c0 // 32), dtype=torch.float32, device="cuda")
            qs0 = torch.empty((1, c0 // 32), dtype=torch.int32, device="cuda")
            y0 = torch.empty((1, r0), dtype=torch.float32, device="cuda")
            call("gx_quantize_q8_0", ctx.ptr, vp(x0d), c0, 1, c0, vp(q0), vp(s0), vp(qs0), None, None)
            # One launch per weight copy, captured once as a HIP graph and
            # replayed: the launches run back to back, not at the pace of
            # Python's calls (a 14 MB product takes less than one call).
            torch.cuda.synchronize()
            cap = torch.cuda.Stream()
            graph = torch.cuda.CUDAGraph()
            call("gx_set_stream", ctx.ptr, ctypes.c_void_p(cap.cuda_stream))
            try:
                with torch.cuda.graph(graph, stream=cap):
                    for i in range(n_copies):
                        call("gx_matmul_q4_0", ctx.ptr, w0s[i].ptr, vp(q0), vp(s0), vp(qs0), None, 1, 0, r0,
                             None, vp(y0), r0)
            finally:
                call("gx_set_stream", ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            replays = 20
            reps = replays * n_copies
            ctx.timer_start()
            for _ in range(replays):
                graph.replay()
            ms0 = ctx.timer_stop() / reps
            b0 = r0 * (c0 // 32) * 18 + c0 + 8 * (c0 // 32) + 4 * r0
            gbs0 = b0 / (ms0 * 1e-3) / 1e9
            extra["c0_q4_0_matvec"] = {"shape": [r0, c0], "M": 1, "kernel_us": round(ms0 * 1e3, 3),
                                       "GB/s": round(gbs0, 1), "hbm_frac": round(gbs0 / HBM_PEAK_GBS, 4),
                                       "bytes_per_launch": b0, "weight_copies": n_copies,
                                       "roofline": {"bound": "hbm", "achieved": round(gbs0, 1),
                                                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                                    "frac": round(gbs0 / HBM_PEAK_GBS, 4),
                                                    "traffic": read_traffic("q4_0_matvec_c0_traffic.txt"),
                                                    "kernel": "q4_0_matvec_kernel"}}
            if args.only == "c0floor":
                extra["c0_floor"] = bench_c0_floor(ctx, torch, graph, n_copies, b0)
            for w_ in w0s:
                w_.free()
            if args.only in ("c0", "c0floor"):
                print(json.dumps(extra))
                return
        w0d = capi.Weight(ctx, w0, capi.Q4_0, r0, c0)
        g2 = synth.rng(2)
        for M in (64, 512, 2048):
            if args.c2_m and M != args.c2_m:
                continue
            x2 = synth.activations(g2, M, c0)
            x2d = dev(x2)
            q2 = torch.empty((M, c0), dtype=torch.int8, device="cuda")
            s2 = torch.empty((M, c0 // 32), dtype=torch.float32, device="cuda")
            qs2 = torch.empty((M, c0 // 32), dtype=torch.int32, device="cuda")
            y2 = torch.empty((M, r0), dtype=torch.float32, device="cuda")
            call("gx_quantize_q8_0", ctx.ptr, vp(x2d), c0, M, c0, vp(q2), vp(s2), vp(qs2), None, None)
            # the int8-MFMA product (every batch's kernel; the fp16-MFMA form
            # is a parity path only)
            for label, q16 in (("i8", None),):
                # warm until ~50 ms of launches have run: the clocks settle
                # under sustained matrix-core load (a 1 ms warm-up left
                # M = 2048 ~15 % slower than the same kernel after others)
                t_w = time.perf_counter()
                while True:
                    for _ in range(5):
                        call("gx_matmul_q4_0", ctx.ptr, w0d.ptr, vp(q2), vp(s2), vp(qs2), vp(q16), M, 0, r0, None,
                             vp(y2), r0)
                    torch.cuda.synchronize()
                    if time.perf_counter() - t_w > 0.05:
                        break
                reps = 50
                ctx.timer_start()
                for _ in range(reps):
                    call("gx_matmul_q4_0", ctx.ptr, w0d.ptr, vp(q2), vp(s2), vp(qs2), vp(q16), M, 0, r0, None,
                         vp(y2), r0)
                ms2 = ctx.timer_stop() / reps
                ops = 2.0 * M * r0 * c0
                tops = ops / (ms2 * 1e-3) / 1e12
                by = r0 * (c0 // 32) * 18 + M * (c0 + 8 * (c0 // 32)) + 4 * M * r0
                extra[f"c2_q4_0_gemm_m{M}_{label}"] = {
                    "shape": [M, r0, c0], "kernel_us": round(ms2 * 1e3, 2), "TOP/s": round(tops, 2),
                    "GMAC/s": round(tops * 1e3 / 2, 1),
                    "int8_mfma_frac": round(tops / INT8_PEAK_TOPS, 4), "GB/s": round(by / (ms2 * 1e-3) / 1e9, 1),
                    "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS,
                                 "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4)}}
        w0d.free()
        if args.only == "c2":
            print(json.dumps(extra))
            return

    if args.only == "valu":
        print(json.dumps(bench_valu(ctx, torch)))
        return
    if args.only == "c3prefill":
        print(json.dumps(bench_c3_prefill(ctx, torch)))
        return
    if args.only == "c3eager":
        print(json.dumps(bench_c3_eager(ctx, torch)))
        return

    # ---- config 3: Qwen3-4B-shaped decoder, prefill 512 + 128 greedy steps ----
    if not args.no_extra and args.only in ("", "c3"):
        extra.update(bench_c3(ctx, torch))
        if args.only == "c3":
            print(json.dumps(extra))
            return

    # ---- config 4: Gemma-shaped MoE layer (route + experts) ----------------
    if not args.no_extra and args.only in ("", "c4"):
        extra.update(bench_c4(ctx, torch, dev))
        if args.only == "c4":
            print(json.dumps(extra))
            return

    # ---- CPU baseline: golem's AVX2 path on this host's cores, and the check --
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w6, x, rows, cols, step_bytes, step, y, torch, args.no_extra)

    traffic = read_traffic("q6_k_matvec_c1_traffic.txt")
    out = {
        "metric": "Q4_0/Q6_K matvec HBM GB/s (% of peak); decode tok/s, Qwen3-4B shape",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded PCG64; Q6_K weights and N(0,1) activations as config 1 specifies)",
        "config": {"workload": "config 1: Q6_K output-head matvec 151936x2560, batch 1, Q8_K activation, "
                               "quantise + product per step, weights rotating over 2 resident copies",
                   "rows": rows, "cols": cols, "batch": 1, "seed": 1},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "q6_k_matvec_kernel", "kernel_us": round(kernel_ms * 1e3, 3),
                     "algorithmic_bytes_per_launch": matvec_bytes},
        "cpu_baseline": cpu,
        "configs": extra,
    }
    print(json.dumps(out))
    for w_ in copies:
        w_.free()
    ctx.close()


def bench_c0_floor(ctx, torch, c0_graph, n_copies, b0):
    """Profiling leg (--only c0floor): config 0's product beside the floors a
    launch of its size meets on this GPU, each a graph of 20 launches
    replayed back to back (as the C0 figure is taken): an empty kernel of 1
    and of 256 workgroups, and a plain 16-byte non-temporal read of C0's
    bytes (rounded to 16) from 20 rotating copies at 152, 304 and 608
    workgroups (the product runs 152, one a 64-row tile).  Per-launch
    microseconds by HIP events; the same leg under rocprofv3 --kernel-trace
    gives the per-dispatch durations."""
    from golem_amd import capi
    import ctypes
    call, vp = capi.call, capi.vp
    nbytes = b0 // 16 * 16
    bufs = [torch.empty((nbytes,), dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(n_copies)]
    sink = torch.zeros((4096,), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()

    def captured(launch):
        torch.cuda.synchronize()
        cap = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        call("gx_set_stream", ctx.ptr, ctypes.c_void_p(cap.cuda_stream))
        try:
            with torch.cuda.graph(g, stream=cap):
                for i in range(n_copies):
                    launch(i)
        finally:
            call("gx_set_stream", ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
        return g

    def per_launch(g, replays=50):
        for _ in range(3):
            g.replay()
        torch.cuda.synchronize()
        ctx.timer_start()
        for _ in range(replays):
            g.replay()
        return ctx.timer_stop() / (replays * n_copies) * 1e3

    out = {"c0_product_us": round(per_launch(c0_graph), 3)}
    for wgs in (1, 256):
        out[f"empty_{wgs}wg_us"] = round(per_launch(captured(lambda i, w=wgs: call("gx_calib_empty", ctx.ptr, w))), 3)
    for wgs in (152, 304, 608):
        us = per_launch(captured(lambda i, w=wgs: call("gx_calib_read", ctx.ptr, vp(bufs[i]), nbytes, w, vp(sink))))
        out[f"read_{wgs}wg_us"] = round(us, 3)
        out[f"read_{wgs}wg_GB/s"] = round(nbytes / (us * 1e-6) / 1e9, 1)
    out["read_bytes"] = nbytes
    out["c0_product_us"] = round(per_launch(c0_graph), 3)  # again, after the others
    return out


def bench_valu(ctx, torch):
    """Profiling leg (--only valu): the VALU-saturating calibration kernel
    (8 independent v_fmac_f32 chains a lane, 2048 workgroups of 256
    threads, 4096 steps), for reading SQ_INSTS_VALU / SQ_ACTIVE_INST_VALU /
    SQ_BUSY_CYCLES of the products against the counters' value at
    saturation."""
    from golem_amd import capi
    call, vp = capi.call, capi.vp
    sink = torch.zeros((4096,), dtype=torch.float32, device="cuda")
    wgs, iters = 2048, 4096
    for _ in range(3):
        call("gx_calib_valu", ctx.ptr, wgs, iters, vp(sink))
    torch.cuda.synchronize()
    ctx.timer_start()
    reps = 10
    for _ in range(reps):
        call("gx_calib_valu", ctx.ptr, wgs, iters, vp(sink))
    ms = ctx.timer_stop() / reps
    fmas = 8.0 * iters * 256 * wgs
    return {"valu": {"workgroups": wgs, "threads": 256, "fmac_per_lane": 8 * iters, "kernel_us": round(ms * 1e3, 2),
                     "wave64_fmac_per_cycle_per_cu_at_2.4GHz": round(fmas / 64 / (ms * 1e-3) / 2.4e9 / 256, 3),
                     "fp32_TFLOP/s": round(2 * fmas / (ms * 1e-3) / 1e12, 1)}}


def cpu_baseline(w6, x, rows, cols, step_bytes, step, y, torch, no_extra):
    """golem's x86 path restated (oracle/cpu_avx2.c: dotQ6_KAVX2 and the
    worker pool of nn/parallel.go) timed on this host: config 1 over two
    rotating weight copies (640 MB, past the last-level cache) for ~10 s on
    every allowed thread and ~3 s on one; the GPU's logits are checked bit for
    bit against it.  Config 0 (Q4_0, dotQ4_0AVX2 under matVecQ4_0Rows) is
    timed the same way for ~3 s, config 2's matrix through golem's packed
    path (dotPackedQ4_0x4AVX2) for ~3 s at each of M = 64, 512 and 2048,
    config 3's whole decode token for ~6 s (cpu_c3_decode) and config 4's
    MoE layer, decode and prefill, ~3 s each (cpu_c4)."""
    import oracle
    threads = oracle.host_threads()
    oracle.cpu_lib(threads)

    def timed(fn, budget):
        fn(0)
        n, t0 = 0, time.perf_counter()
        while True:
            fn(n)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return n, el

    b = oracle.Batch(x).quantize_k()
    hw = [w6, w6.copy()]
    yc = np.zeros((1, rows), dtype=np.float32)
    n_all, t_all = timed(lambda i, th=threads: oracle.cpu_mat_vec_q6_k(hw[i & 1], b, rows, th, yc), 10.0)
    n_one, t_one = timed(lambda i: oracle.cpu_mat_vec_q6_k(hw[i & 1], b, rows, 1, yc), 3.0)
    oracle.cpu_mat_vec_q6_k(w6, b, rows, threads, yc)
    step(0)  # recompute on copy 0 for the bit-for-bit check
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    exact = bool(np.array_equal(got.view(np.uint32), yc.view(np.uint32)))
    out = {"value": round(n_all * step_bytes / t_all / 1e9, 2), "unit": "GB/s", "cores": threads, "kind": "port",
           "sample": f"{n_all} passes of config 1 (151936x2560 Q6_K, M=1) through golem's AVX2 Q6_K kernel and "
                     f"worker pool restated in C, {threads} threads, 2 rotating weight copies, {t_all:.1f} s",
           "one_thread_value": round(n_one * step_bytes / t_one / 1e9, 2),
           "gpu_logits_bit_exact": exact}
    if not no_extra:
        from golem_amd import synth
        r0, c0 = 9728, 2560
        g0 = synth.rng(0)
        w0 = synth.q4_0_weights(g0, r0, c0)
        b0 = oracle.Batch(synth.activations(g0, 1, c0)).quantize()
        h0 = [w0] + [w0.copy() for _ in range(19)]
        y0 = np.zeros((1, r0), dtype=np.float32)
        n0, t0 = timed(lambda i: oracle.cpu_mat_vec_q4_0(h0[i % 20], b0, r0, threads, y0), 3.0)
        by0 = r0 * (c0 // 32) * 18 + c0 + 8 * (c0 // 32) + 4 * r0
        out["c0_q4_0_matvec"] = {"GB/s": round(n0 * by0 / t0 / 1e9, 2), "us_per_pass": round(t0 / n0 * 1e6, 1),
                                 "cores": threads, "passes": n0}
        # Config 2 (Q4_0 9728 x 2560 against M tokens) through golem's packed
        # path (PackQ4_0's eight-row groups, dotPackedQ4_0x4AVX2 under
        # matVecPackedQ4_0Rows): ~3 s each at M = 64 and 512.
        packed = oracle.pack_q4_0(w0, r0, c0)
        g2 = synth.rng(2)
        for M in (64, 512, 2048):
            b2 = oracle.Batch(synth.activations(g2, M, c0)).quantize()
            y2 = np.zeros((M, r0), dtype=np.float32)
            n2, t2 = timed(lambda i: oracle.cpu_mat_vec_packed_q4_0(packed, b2, r0, threads, y2), 3.0)
            macs = float(M) * r0 * c0
            out[f"c2_q4_0_packed_m{M}"] = {"GMAC/s": round(n2 * macs / t2 / 1e9, 2),
                                           "ms_per_pass": round(t2 / n2 * 1e3, 2), "cores": threads, "passes": n2}
        out["c3_decode_token"] = cpu_c3_decode(oracle, synth, w6, timed, threads)
        out.update(cpu_c4(oracle, synth, timed, threads))
    return out


def cpu_c3_decode(oracle, synth, w6, timed, threads):
    """Config 3's whole decode token on the CPU, golem's x86 engine restated
    (oracle/cpu_avx2.c cpu_qwen_token: per block the pre-norms and their
    Q8_0, the head section -- Q/K/V rows through matVecPackedQ4_0Rows, head
    norms, RoPE, fp16 rounding, the cache store --, the attention section --
    dotF32AVX2 scores, SoftmaxInPlace, fp16 probabilities, Axpy, the heads'
    Q8_0 --, O, the FFN section -- Gate and Up rows, SwiGLU, Q8_0 --, Down,
    the residual adds; then the final norm, QuantizeK and the Q6_K head),
    36 blocks with their own packed weights (2 GB, past the last-level
    cache), caches of fp16-rounded values, positions 576 .. 639 in turn."""
    from golem_amd.qwen import rope_tables
    cfg = synth.qwen3_4b(640)
    g = synth.rng(3)
    one = synth.qwen_weights(synth.QwenConfig(cfg.dim, cfg.ffn, 1, cfg.heads, cfg.kv_heads, cfg.head_dim, 256,
                                              cfg.max_context), 3)
    w = {"blocks": [one["blocks"][0]] * cfg.layers, "output_norm": one["output_norm"], "token_embd": w6}
    cpu = oracle.CpuQwen(cfg, w)
    for kc, vc in cpu.caches:
        kc[:] = g.standard_normal(kc.shape).astype(np.float16)
        vc[:] = g.standard_normal(vc.shape).astype(np.float16)
    cos, sin = rope_tables(cfg.head_dim, cfg.max_context, cfg.rope_base)
    x0 = synth.activations(g, 1, cfg.dim)[0]

    def token(i):
        pos = 576 + i % 64
        cpu.token(x0.copy(), pos, cos[pos], sin[pos], threads)

    n, t = timed(token, 6.0)
    del cpu
    return {"tok_per_s": round(n / t, 2), "ms_per_token": round(t / n * 1e3, 1), "cores": threads, "tokens": n,
            "scope": "a whole decode token (36 blocks: norms, products, head norms, RoPE, cache, attention over "
                     "577..640 positions, SwiGLU; final norm and Q6_K head), golem's x86 engine restated"}


def cpu_c4(oracle, synth, timed, threads):
    """Config 4 on the CPU: gemma's Route + ExpertFFN through golem's x86
    kernels (oracle/cpu_avx2.c cpu_moe_ffn: dotF32AVX2 router, the
    worker-pool sections over positions and (position, slot) units, the
    expert stacks in the row layout through matVecQ4_0Rows), decode (one
    position, 64 different inputs in turn) and the 256-position prefill, on
    config 4's seeded weights (428 MB of experts)."""
    D, F, E, k = 2816, 704, 128, 8
    g = synth.rng(4)
    router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    gate_up = synth.q4_0_weights(g, E * 2 * F, D)
    down = synth.q4_0_weights(g, E * D, F)
    expert_bytes = (2 * F * (D // 32) + D * (F // 32)) * 18
    out = {}
    for label, M, npos in (("decode", 1, 64), ("prefill256", 256, 2)):
        xs = [synth.activations(g, M, D) for _ in range(npos)]
        moe = oracle.CpuMoE(router, gate_up, down, D, F, E, k, M)
        touched = [len(np.unique(moe.run(x, threads)[1])) for x in xs]
        n, t = timed(lambda i: moe.run(xs[i % npos], threads), 3.0)
        ms = t / n * 1e3
        by = float(np.mean(touched)) * expert_bytes + E * D * 4
        out[f"c4_moe_{label}"] = {"ms_per_layer": round(ms, 3), "positions_per_s": round(M / (ms * 1e-3), 1),
                                  "GB/s": round(by / (ms * 1e-3) / 1e9, 2), "cores": threads, "passes": n}
    return out


def bench_c3_prefill(ctx, torch):
    """Profiling leg: config 3's model and 512-token prompt (as bench_c3),
    the prompt read four times from an empty cache, each timed with HIP
    events through its first token."""
    from golem_amd import synth
    from golem_amd.qwen import QwenModel
    cfg = synth.qwen3_4b(640)
    w = synth.qwen_weights(cfg, 3)
    model = QwenModel(ctx, cfg, w, max_batch=512)
    del w
    prompt = synth.rng(3).integers(0, cfg.vocab, 512).astype(np.int32)
    ms = []
    for _ in range(4):
        model.reset()
        torch.cuda.synchronize()
        ctx.timer_start()
        model.forward(prompt, 0)
        model.next_token(len(prompt) - 1)
        ms.append(round(ctx.timer_stop(), 3))
    return {"c3_prefill_ms": ms}


def bench_c3_eager(ctx, torch):
    """Profiling leg for counter passes (rocprofv3 --pmc does not survive
    this leg's graph capture): config 3's model and prompt, then 24 decode
    steps launched eagerly, one position at a time -- the same kernels and
    shapes as the captured step, each launch on its own."""
    from golem_amd import synth
    from golem_amd.qwen import QwenModel
    cfg = synth.qwen3_4b(640)
    w = synth.qwen_weights(cfg, 3)
    model = QwenModel(ctx, cfg, w, max_batch=512)
    del w
    prompt = synth.rng(3).integers(0, cfg.vocab, 512).astype(np.int32)
    model.reset()
    model.forward(prompt, 0)
    tok = int(model.next_token(len(prompt) - 1).item())
    ids = [tok]
    ctx.timer_start()
    for s in range(24):
        model.forward([tok], len(prompt) + s)
        tok = int(model.next_token(0).item())
        ids.append(tok)
    ms = ctx.timer_stop() / 24
    model.free()
    return {"c3_eager_decode_ms_per_token": round(ms, 3), "ids": ids[:8]}


def bench_c3(ctx, torch):
    """Config 3: Qwen3-4B's shape (36 blocks, 2560 wide, FFN 9728, 32/8 heads of
    128, vocab 151936) with random weights drawn as config 3 specifies (seed
    3): a 512-token prompt of uniform random ids read in one batch, then 128
    greedy tokens, each fed back from the device, with the fp16 cache growing
    to 640; the decode steps are replays of one captured HIP graph.  Timed
    with HIP events: the prefill (through the first token) and the 127 decode
    steps after it."""
    from golem_amd import synth
    from golem_amd.qwen import QwenModel
    cfg = synth.qwen3_4b(640)
    t0 = time.perf_counter()
    w = synth.qwen_weights(cfg, 3)
    model = QwenModel(ctx, cfg, w, max_batch=512)
    del w
    torch.cuda.synchronize()
    setup_s = time.perf_counter() - t0
    prompt = synth.rng(3).integers(0, cfg.vocab, 512).astype(np.int32)
    model.reset()
    model.forward(prompt[:16], 0)
    model.start_decode(model.next_token(15), 16)
    model.capture_decode()
    for _ in range(3):
        model.graph.replay()
    torch.cuda.synchronize()

    # one untimed prefill first: the clocks settle under the products'
    # sustained matrix-core load, and the timed one is the steady state
    model.reset()
    model.forward(prompt, 0)
    model.next_token(len(prompt) - 1)
    model.reset()
    torch.cuda.synchronize()
    ctx.timer_start()
    model.forward(prompt, 0)
    tok = model.next_token(len(prompt) - 1)
    prefill_ms = ctx.timer_stop()
    steps = 128
    ctx.timer_start()
    model.start_decode(tok, len(prompt))
    for s in range(steps - 1):
        model.graph.replay()
    decode_ms = ctx.timer_stop()
    ids = model.decoded(len(prompt), steps)
    q4 = lambda r, c: r * (c // 32) * 18
    qd, kvd = cfg.heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    layer_bytes = (q4(qd + 2 * kvd, cfg.dim) + q4(cfg.dim, qd) + q4(2 * cfg.ffn, cfg.dim) + q4(cfg.dim, cfg.ffn))
    head_bytes = cfg.vocab * (cfg.dim // 256) * 210
    mean_ctx = len(prompt) + steps / 2
    kv_bytes = cfg.layers * mean_ctx * cfg.kv_heads * cfg.head_dim * 2 * 2
    token_bytes = cfg.layers * layer_bytes + head_bytes + kv_bytes
    per_tok = decode_ms / (steps - 1)

    # Eight conversations decoded in lock step (slots): one pass over the
    # weights and one head read per step for all eight.
    nconv, slot_prompt, slot_steps = 8, 64, 16
    model.set_slots(nconv)
    firsts = []
    for i in range(nconv):
        model.use_slot(i)
        model.forward(prompt[i * slot_prompt:(i + 1) * slot_prompt], 0)
        firsts.append(int(model.next_token(slot_prompt - 1).item()))
    slot_ms = {}
    for graph in (False, True):  # eager steps, then replays of the captured step
        model.start_slots(firsts, [slot_prompt] * nconv)
        model.slots_step(nconv, graph=graph)  # warm (and, for the graph, its capture)
        model.start_slots(firsts, [slot_prompt] * nconv)
        torch.cuda.synchronize()
        ctx.timer_start()
        for _ in range(slot_steps):
            model.slots_step(nconv, graph=graph)
        slot_ms[graph] = ctx.timer_stop() / slot_steps
    slot_step_ms = slot_ms[True]
    model.free()
    return {"c3_qwen3_4b_slots": {
        "conversations": nconv, "prompt_each": slot_prompt, "steps": slot_steps,
        "ms_per_step": round(slot_step_ms, 3), "tok_per_s": round(nconv * 1e3 / slot_step_ms, 1),
        "graph": True, "eager_ms_per_step": round(slot_ms[False], 3)},
        "c3_qwen3_4b": {
        "prefill_tokens": len(prompt), "prefill_ms": round(prefill_ms, 2),
        "prefill_tok_per_s": round(len(prompt) / (prefill_ms * 1e-3), 1),
        "decode_steps": steps, "decode_ms_per_token": round(per_tok, 3),
        "decode_tok_per_s": round(1e3 / per_tok, 1),
        "decode_bytes_per_token": int(token_bytes),
        "decode_GB/s": round(token_bytes / (per_tok * 1e-3) / 1e9, 1),
        "decode_hbm_frac": round(token_bytes / (per_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": round(token_bytes / (per_tok * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(token_bytes / (per_tok * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                     "scope": "a whole decode step (every kernel), bytes a token reads"},
        "greedy_ids_head": ids[:8], "setup_s": round(setup_s, 1)}}


def bench_c4(ctx, torch, dev):
    """Config 4: router (128 x 2816 fp32) + top-8 + 8 GELU-gated Q4_0 experts
    per position (gate_up 1408 x 2816, down 2816 x 704), seed 4. Decode (one
    position) and a 256-position prefill grouped by expert, each timed as
    route + experts with HIP events (decode also as replays of a captured
    graph of 16 steps, the figure reported; the eager figure beside it). Two
    copies of the expert stacks (856 MB, beyond the 256 MB last-level cache)
    alternate between steps, and decode walks 64 different positions, so the
    experts a step reads are not cached."""
    from golem_amd import capi, synth
    import ctypes
    call, vp = capi.call, capi.vp
    D, F, E, k = 2816, 704, 128, 8
    g = synth.rng(4)
    router = (g.standard_normal((E, D)) * 0.02).astype(np.float32)
    gate_up = synth.q4_0_weights(g, E * 2 * F, D)
    down = synth.q4_0_weights(g, E * D, F)
    wr = capi.Weight(ctx, router, capi.F32, E, D)
    stacks = [(capi.Weight(ctx, gate_up, capi.Q4_0, 2 * F, D, count=E),
               capi.Weight(ctx, down, capi.Q4_0, D, F, count=E)) for _ in range(2)]
    expert_bytes = (2 * F * (D // 32) + D * (F // 32)) * 18
    res = {}
    for label, M, npos in (("decode", 1, 64), ("prefill256", 256, 2)):
        xs = [dev(synth.activations(g, M, D)) for _ in range(npos)]
        logits = torch.empty((M, E), dtype=torch.float32, device="cuda")
        ids = torch.empty((M, k), dtype=torch.int32, device="cuda")
        wts = torch.empty((M, k), dtype=torch.float32, device="cuda")
        out = torch.empty((M, D), dtype=torch.float32, device="cuda")
        n = ctypes.c_size_t()
        call("gx_moe_workspace_bytes", M, k, D, F, E, ctypes.byref(n))
        ws = torch.empty((n.value,), dtype=torch.uint8, device="cuda")

        def step(i):
            x = xs[i % npos]
            gu, dn = stacks[i & 1]
            call("gx_moe_route", ctx.ptr, wr.ptr, None, vp(x), D, M, k, np.float32(1e-6), vp(logits), vp(ids),
                 vp(wts))
            call("gx_moe_experts", ctx.ptr, gu.ptr, dn.ptr, None, vp(x), D, M, k, vp(ids), vp(wts), vp(out), D,
                 vp(ws), n.value)

        # warm until ~50 ms of steps have run (the clocks settle under load)
        t_w, i = time.perf_counter(), 0
        while i < 6 or time.perf_counter() - t_w < 0.05:
            step(i)
            i += 1
            if i % 8 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        # distinct experts each position set reads, for the algorithmic bytes
        touched = []
        for i in range(npos):
            step(i)
            torch.cuda.synchronize()
            touched.append(len(np.unique(ids.cpu().numpy())))
        reps = 128 if M == 1 else 20
        ctx.timer_start()
        for i in range(reps):
            step(i)
        ms = ctx.timer_stop() / reps
        eager_ms = ms
        if M == 1:
            # Decode as a serving loop runs it: the layer's launches captured
            # once (16 steps over rotating inputs and stacks) and replayed.
            gsteps = 16
            torch.cuda.synchronize()
            stream = torch.cuda.Stream()
            graph = torch.cuda.CUDAGraph()
            call("gx_set_stream", ctx.ptr, ctypes.c_void_p(stream.cuda_stream))
            try:
                with torch.cuda.graph(graph, stream=stream):
                    for i in range(gsteps):
                        step(i)
            finally:
                call("gx_set_stream", ctx.ptr, None)
            for _ in range(2):
                graph.replay()
            torch.cuda.synchronize()
            greps = 8
            ctx.timer_start()
            for _ in range(greps):
                graph.replay()
            ms = ctx.timer_stop() / (greps * gsteps)
            del graph
        mean_touched = float(np.mean(touched))
        by = mean_touched * expert_bytes + E * D * 4 + M * D * 4 * 2
        res[f"c4_moe_{label}"] = {
            "M": M, "ms_per_layer": round(ms, 4), "positions_per_s": round(M / (ms * 1e-3), 1),
            "experts_read": round(mean_touched, 2), "bytes_per_layer": int(by),
            "GB/s": round(by / (ms * 1e-3) / 1e9, 1), "hbm_frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "graph": M == 1, "eager_ms_per_layer": round(eager_ms, 4),
            "roofline": {"bound": "hbm", "achieved": round(by / (ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "scope": "the layer's launches (route + experts), bytes of the experts read"}}
    wr.free()
    for gu, dn in stacks:
        gu.free()
        dn.free()
    res.update(bench_c4_moe_half(ctx, torch, dev))
    return res


def bench_c4_moe_half(ctx, torch, dev):
    """The whole feed-forward half of the mixture block (moeHalf): the shared
    dense branch, the router and experts, and the three post-norms, config
    4's experts and router.  Config 4 gives no width for the shared branch;
    the hidden width (2816) is used.  Decode (M = 1) and a 256-position
    prefill; the residual norm under ffn_norm is included."""
    from golem_amd import synth
    from golem_amd.gemma import MoEConfig, MoEHalf, moe_weights
    cfg = MoEConfig(2816, 2816, 128, 8, 704)
    g = synth.rng(4)
    w = moe_weights(cfg, g)
    blk = MoEHalf(ctx, cfg, w, max_batch=256)
    res = {}
    for label, M, npos in (("decode", 1, 64), ("prefill256", 256, 2)):
        xs = [dev(synth.activations(g, M, cfg.dim)) for _ in range(npos)]
        out = torch.empty((M, cfg.dim), dtype=torch.float32, device="cuda")
        for i in range(4):
            blk.forward(xs[i % npos], out)
        torch.cuda.synchronize()
        reps = 64 if M == 1 else 10
        ctx.timer_start()
        for i in range(reps):
            blk.forward(xs[i % npos], out)
        ms = ctx.timer_stop() / reps
        res[f"c4_moe_half_{label}"] = {"M": M, "ms_per_layer": round(ms, 4),
                                       "positions_per_s": round(M / (ms * 1e-3), 1), "shared_ffn": cfg.ffn}
    blk.free()
    return res


if __name__ == "__main__":
    main()
