"""Benchmark of the quantized matmul path on one MI355X (prints ONE JSON line).

Metric: IQ4_XS GEMV weight GB/s (decode) + int8 GEMM TOPS (2K prompt), % of peak.
  value     -- IQ4_XS decode GEMV weight GB/s. A step is one decode pass over the two 27B-class FFN matrices,
               K=5120 -> N=17408 (gate/up) and K=17408 -> N=5120 (down), batch 1, weights resident in HBM and
               rotated over 8 distinct copies of each matrix (758 MB > the 256 MB Infinity Cache).
  gemm      -- the 2K-token prompt GEMM: Q4_K weights K=5120, N=17408, M=2048 int8 activations, int8 MFMA;
               TOPS = 2*M*N*K / time.
  moe       -- the MoE FFN (256 experts, E 2048, F 512, T 4096, top-8, Zipf 1.1 router, IQ4_XS), reported.
  reported  -- the other BASELINE configs (Q8_0 4096x4096 GEMV; IQ3_S 5120x5120 GEMV at M=1 and GEMM at M=512)
               and the activation producers that feed the path (rmsnorm_quant, swiglu_quant, add_norm_quant).
  roofline  -- for each kernel: algorithmic bytes (or int8 ops) per launch / average launch time, measured with
               HIP events on the launch stream, against MI355X peaks (HBM 8 TB/s, dense int8 MFMA 5.0 POPS).
  cpu_baseline -- the repository's C restatement of the reference CPU path (oracle/), timed on this host.
"""
import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
METRIC = "IQ4_XS GEMV weight GB/s (decode) + int8 GEMM TOPS (2K prompt), % of peak"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    # (2000 warm-up steps, ~50 ms of GEMV work: the GPU's clocks settle under load within tens of milliseconds; with 20
    #  the timed steps ran ~15 % slower while the clocks were still rising)
    p.add_argument("--warmup", type=int, default=2000)
    # (the GPU's clocks rise over tens of milliseconds of load: each leg first replays its warm-up untimed for at
    #  least this long, whatever --warmup says, so short warm-ups do not time a GPU that is still clocking up)
    p.add_argument("--settle-ms", type=float, default=300.0)
    p.add_argument("--only", choices=["all", "gemv", "gemm", "moe", "report"], default="all")
    p.add_argument("--copies", type=int, default=8)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=8.0, help="CPU work budget per baseline leg")
    p.add_argument("--profile", action="store_true",
                   help="short run for rocprofv3: a few launches of each kernel plus a 1 GiB copy for calibration")
    return p.parse_args()


SETTLE_S = 0.3


def settle(fn):
    """Run fn untimed until SETTLE_S seconds of wall time have passed (at least once)."""
    import torch
    t0 = time.perf_counter()
    while True:
        fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= SETTLE_S:
            return


def timed(fn, steps, warmup, stream, pre=None):
    import torch
    if SETTLE_S > 0:
        settle(lambda: [fn(i) for i in range(max(1, warmup))])
    for i in range(warmup):
        fn(i)
    if pre is not None:
        pre()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(end) / steps, wall


def graphed(fn, n):
    """fn(0..n-1) captured once into a HIP graph (torch.cuda.CUDAGraph on ROCm)."""
    import torch
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(n):
            fn(i)
    return g


def timed_graph(fn, args, stream):
    """W warmup steps, then exactly K timed steps, each captured once and replayed: short launches (a batch-1 GEMV is
    ~10 us of GPU time, about what a Python-side launch costs) would otherwise time the host."""
    import torch
    for i in range(2):
        fn(i)  # (first-launch work stays out of the captures)
    torch.cuda.synchronize()
    gw, gt = graphed(fn, max(1, args.warmup)), graphed(fn, args.steps)
    if SETTLE_S > 0:
        settle(gw.replay)
    ms, _ = timed(lambda i: gt.replay(), 1, 0, stream, pre=gw.replay)
    return ms / args.steps


def timed_graph_n(fn, n, stream):
    """fn(0..n-1) captured once and replayed (a warm-up replay, the settle time, then one timed replay); ms per call."""
    import torch
    for i in range(2):
        fn(i)
    torch.cuda.synchronize()
    g = graphed(fn, n)
    if SETTLE_S > 0:
        settle(g.replay)
    ms, _ = timed(lambda i: g.replay(), 1, 0, stream, pre=g.replay)
    return ms / n


def profile_traffic(kernel_key):
    """Bytes per launch from the committed rocprofv3 --pmc summaries (FETCH_SIZE + WRITE_SIZE, calibrated on a copy
    kernel), or None."""
    path = os.path.join(ROOT, "profiles", "traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        m = re.match(r"^TRAFFIC\s+(\S+)\s+bytes_per_launch=(\d+)", line)
        if m and m.group(1) == kernel_key:
            return int(m.group(2))
    return None


def main():
    args = parse()
    global SETTLE_S
    SETTLE_S = 0.0 if args.profile else args.settle_ms / 1e3
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported (sharding across GPUs is "
              "designed but not built: every box here has one GPU)", file=sys.stderr)
        sys.exit(2)
    import numpy as np
    import torch

    from arcinfer_amd import formats as F
    from arcinfer_amd import qmatmul as qm

    qm.load_library()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    out = {"metric": METRIC, "value": None, "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": None, "settle_ms": args.settle_ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8",
           "data": "synthetic (seeded GGUF-format weights, N(0,1) activations; BASELINE.json configs)",
           "config": {"workload": "IQ4_XS decode GEMV, batch 1: K=5120->N=17408 and K=17408->N=5120 per step, "
                                  f"{args.copies} rotating weight copies each", "parallelism": "none (1 GPU)"}}
    nthreads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    if args.profile:
        args.steps, args.warmup, args.copies = 4, 1, 2

    # ---------------- IQ4_XS decode GEMV (north star)
    if args.only in ("all", "gemv"):
        shapes = [(17408, 5120), (5120, 17408)]
        mats = []
        for si, (N, K) in enumerate(shapes):
            W = F.synth_weight(F.IQ4_XS, N, K, seed=1 + si)
            Wd = torch.from_numpy(W).to(dev)
            copies = [qm.QWeight(F.IQ4_XS, Wd, N, K) for _ in range(args.copies)]
            del Wd
            x = torch.from_numpy(F.synth_activations(1, K, seed=1 + si)).to(dev)
            aq, asc, absum = qm.quantize_act(x, M_stride=16)
            C = torch.empty((1, N), device=dev)
            mats.append((N, K, W, copies, aq, asc, absum, C))
        torch.cuda.synchronize()
        bytes_per_step = sum(F.weight_bytes(F.IQ4_XS, N, K) for N, K, *_ in mats)

        def step(i):
            for N, K, W, copies, aq, asc, absum, C in mats:
                qm.gemv(copies[i % len(copies)], aq, asc, absum, C=C, ldc=N)

        ms = timed_graph(step, args, stream)
        gbs = bytes_per_step / (ms * 1e-3) / 1e9
        out["value"] = round(gbs, 1)
        out["ms_per_step"] = round(ms, 5)
        # per-matrix launch times (each kernel alone, same rotation)
        per = {}
        for N, K, W, copies, aq, asc, absum, C in mats:
            def one(i, copies=copies, aq=aq, asc=asc, absum=absum, C=C, N=N):
                qm.gemv(copies[i % len(copies)], aq, asc, absum, C=C, ldc=N)
            ms1 = timed_graph(one, args, stream)
            b = F.weight_bytes(F.IQ4_XS, N, K)
            per[f"{K}->{N}"] = {"us_per_launch": round(ms1 * 1e3, 2), "GB/s": round(b / (ms1 * 1e-3) / 1e9, 1),
                               "weight_bytes": b}
        out["gemv_per_matrix"] = per
        # multi-token decode GEMV (T tokens against one weight read: speculative verification), gate/up matrix
        N, K, W, copies, aq1, asc1, absum1, C1 = mats[0]
        mt = {}
        for T in (2, 4, 8):
            xT = torch.from_numpy(F.synth_activations(T, K, seed=7 + T)).to(dev)
            aqT, ascT, absT = qm.quantize_act(xT, M_stride=16)
            CT = torch.empty((T, N), device=dev)

            def oneT(i, aqT=aqT, ascT=ascT, absT=absT, CT=CT, T=T):
                qm.gemv(copies[i % len(copies)], aqT, ascT, absT, T=T, C=CT, ldc=N)
            msT = timed_graph(oneT, args, stream)
            b = F.weight_bytes(F.IQ4_XS, N, K)
            mt[str(T)] = {"us_per_launch": round(msT * 1e3, 2), "weight_GB/s": round(b / (msT * 1e-3) / 1e9, 1)}
        out["gemv_multi_token_5120->17408"] = mt
        # the dominant kernel of the step: the matrix whose launch takes longer (the down projection, K 17408 -> N 5120,
        # at this build's kernels); both matrices' fractions and the whole step's are reported beside it
        dom_key = max(per, key=lambda k: per[k]["us_per_launch"])
        dom = per[dom_key]
        Kd, Nd = (int(v) for v in dom_key.split("->"))
        lpr = 32 if Kd // 32 <= 256 and Nd > 6144 else 128  # (the batch-1 route of qm_gemv_impl.h)
        traffic = profile_traffic(f"gemv_iq4_xs_{Kd}x{Nd}")
        out["roofline"] = {"bound": "hbm",
                           "kernel": f"gemvs_kernel (IQ4_XS, {lpr} lanes per row) K={Kd} N={Nd}: the step's longer launch",
                           "achieved": dom["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                           "frac": round(dom["GB/s"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                           "algorithmic_bytes_per_launch": dom["weight_bytes"],
                           "per_matrix_frac": {k: round(v["GB/s"] / HBM_PEAK_GBS, 4) for k, v in per.items()},
                           "step_frac": round(gbs / HBM_PEAK_GBS, 4)}
        out["gemv_frac_of_hbm_peak"] = round(gbs / HBM_PEAK_GBS, 4)
        if not args.no_cpu and not args.profile:
            import oracle
            N, K, W, copies, aq, asc, absum, C = mats[0]
            naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
            reps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < args.cpu_seconds:
                oracle.blockdot(F.IQ4_XS, W, K, naq, nasc, nabs, M=1, nthreads=nthreads)
                reps += 1
            cpu_s = (time.perf_counter() - t0) / reps
            out["cpu_baseline"] = {"value": round(F.weight_bytes(F.IQ4_XS, N, K) / cpu_s / 1e9, 3), "unit": "GB/s",
                                   "cores": nthreads, "kind": "port",
                                   "sample": f"IQ4_XS K=5120 N=17408 int8 block-dot GEMV (oracle/qref.c, -O3, "
                                             f"OpenMP), {reps} full passes in {reps * cpu_s:.1f} s"}
        for m in mats:
            for c in m[3]:
                c.release()
        del mats
        torch.cuda.empty_cache()

    # ---------------- Q4_K prompt GEMM, 2048 tokens
    if args.only in ("all", "gemm"):
        M, N, K = 2048, 17408, 5120
        W = F.synth_weight(F.Q4_K, N, K, seed=2)
        w = qm.QWeight(F.Q4_K, torch.from_numpy(W).to(dev), N, K)
        x = torch.from_numpy(F.synth_activations(M, K, seed=2, outlier_frac=0.01, outlier_scale=20.0)).to(dev)
        aq, asc, absum = qm.quantize_act(x)
        C = torch.empty((M, N), device=dev)
        steps = max(2, args.steps // 5)
        # (timed from a replayed HIP graph of the allocation-free entry, which runs the same kernels as qmatmul_gemm:
        #  the activation prepass and the f16-MFMA GEMM)
        gargs = argparse.Namespace(**{**vars(args), "steps": steps})
        ms = timed_graph(lambda i: qm.gemm(w, aq, asc, absum, C=C, ldc=N, noalloc=True), gargs, stream)
        ops = 2.0 * M * N * K
        tops = ops / (ms * 1e-3) / 1e12
        g = {"value": round(tops, 1), "unit": "TOPS", "ms_per_launch": round(ms, 4),
             "config": "Q4_K K=5120 N=17408, M=2048 (1% outlier channels x20), int8 per-32 activations",
             "roofline": {"bound": "mfma", "kernel": "f16_act_kernel + gemm_f16_kernel<12> (Q4_K as exact f16 sc*q, "
                                                     "128 x 128 tiles; the int8-op count of the product over the "
                                                     "dense int8 peak)", "achieved": round(tops, 1),
                          "peak": INT8_PEAK_TOPS, "unit": "TOP/s", "frac": round(tops / INT8_PEAK_TOPS, 4),
                          "traffic": profile_traffic("gemm_q4_k_2048x5120x17408"),
                          "algorithmic_ops_per_launch": int(ops)}}
        # activation quantizer for the same 2048 x 5120 input (the step before the GEMM)
        msq, _ = timed(lambda i: qm.quantize_act(x), steps, 1, stream)
        g["quantize_us"] = round(msq * 1e3, 2)
        if not args.no_cpu and not args.profile:
            import oracle
            naq, nasc, nabs = aq.cpu().numpy(), asc.cpu().numpy(), absum.cpu().numpy()
            stride = 64
            t0 = time.perf_counter()
            oracle.blockdot(F.Q4_K, W, K, naq, nasc, nabs, col_stride=stride, nthreads=nthreads)
            cpu_s = (time.perf_counter() - t0) * stride
            g["cpu_baseline"] = {"value": round(ops / cpu_s / 1e12, 4), "unit": "TOPS", "cores": nthreads,
                                 "kind": "port", "sample": f"every {stride}th output column of the same GEMM "
                                                           f"(oracle/qref.c int8 block-dot), time x {stride}"}
            # the other two CPU paths of the reference: the activation quantizer (quantize_act_cpu, one thread)
            # and the f32 dequantize-and-multiply reference (tools/ref_forward.cpp matmul: dequant_row + dot)
            xh = x.cpu().numpy()
            t0 = time.perf_counter()
            oracle.quantize_act(xh)
            q_s = time.perf_counter() - t0
            Ms_ = 64
            t0 = time.perf_counter()
            oracle.matmul_f32(F.Q4_K, W, K, xh[:Ms_], nthreads=nthreads)
            f_s = time.perf_counter() - t0
            g["cpu_baseline_other_paths"] = {
                "quantize_act": {"us": round(q_s * 1e6, 1), "cores": 1, "kind": "port",
                                 "sample": "the same 2048 x 5120 f32 activations (oracle/qref.c)",
                                 "gpu_us": g["quantize_us"]},
                "matmul_f32": {"value": round(2.0 * Ms_ * N * K / f_s / 1e12, 5), "unit": "TFLOP/s", "cores": nthreads,
                               "kind": "port",
                               "sample": f"the first {Ms_} tokens of the same GEMM, f32 dequantized weights, f64 dots"}}
        # the same Q4_K GEMM with per-256 activation scales (the reference's act32 = false layout, qmatmul_gemm_ex):
        # one scale per token and superblock, so the f16 MFMAs accumulate the superblock and no per-block VALU scaling
        # runs (reported beside the per-32 headline; the inputs are this x quantized per 256)
        aq2, asc2, absum2 = qm.quantize_act(x, act32=False)
        ms2, _ = timed(lambda i: qm.gemm(w, aq2, asc2, absum2, C=C, ldc=N, act32=False), steps, args.warmup, stream)
        g["act32_false"] = {"TOPS": round(ops / (ms2 * 1e-3) / 1e12, 1), "ms_per_launch": round(ms2, 4),
                            "frac_of_int8_peak": round(ops / (ms2 * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4)}
        del aq2, asc2, absum2
        # the same prompt GEMM with Q6_K weights (per-16 scales: two K=16 MFMAs per block), reported
        W6 = F.synth_weight(F.Q6_K, N, K, seed=6)
        w6 = qm.QWeight(F.Q6_K, torch.from_numpy(W6).to(dev), N, K)
        ms6, _ = timed(lambda i: qm.gemm(w6, aq, asc, absum, C=C, ldc=N), steps, args.warmup, stream)
        g["q6_k"] = {"TOPS": round(ops / (ms6 * 1e-3) / 1e12, 1), "ms_per_launch": round(ms6, 4)}
        w6.release()
        out["gemm"] = g
        w.release()
        del C, x, aq, asc, absum
        torch.cuda.empty_cache()

    # ---------------- MoE FFN (reported)
    if args.only in ("all", "moe"):
        NE, E, Fd, T, NU = 256, 2048, 512, 4096, 8
        ws_ = []
        for i, (rows, K) in enumerate(((NE * Fd, E), (NE * Fd, E), (NE * E, Fd))):
            W = F.synth_weight(F.IQ4_XS, rows, K, seed=40 + i, sigma=0.05)
            ws_.append(qm.QWeight(F.IQ4_XS, torch.from_numpy(W).to(dev), rows, K))
            del W
        x = torch.from_numpy(F.synth_activations(T, E, seed=43)).to(dev)
        aq, asc, absum = qm.quantize_act(x)
        lg = torch.from_numpy(F.zipf_router_logits(T, NE, seed=44)).to(dev)
        wsp = qm.moe_workspace(T, NE, NU, E, Fd, device=dev)
        xo = torch.empty((T, E), device=dev)
        # (timed from a replayed HIP graph, like the other legs: route, scan, scatter, gate/up, down and combine launches
        #  captured once; 20 warm-up and 40 timed layers)
        gargs = argparse.Namespace(**{**vars(args), "steps": 4 if args.profile else 40,
                                      "warmup": 1 if args.profile else 20})
        ms = timed_graph(lambda i: qm.moe_grouped(ws_[0], ws_[1], ws_[2], NE, lg, NU, aq, asc, xo, wsp), gargs, stream)
        ops = 2.0 * T * NU * (2 * Fd * E + E * Fd)
        wbytes = 3 * F.weight_bytes(F.IQ4_XS, NE * Fd, E)
        out["moe"] = {"ms_per_launch": round(ms, 4), "TOPS": round(ops / (ms * 1e-3) / 1e12, 2),
                      "expert_weight_GB/s": round(wbytes / (ms * 1e-3) / 1e9, 1),
                      "config": "256 experts IQ4_XS, E 2048, F 512, T 4096, top-8, Zipf(1.1) router; "
                                "route + scan + scatter + gate/up + down + combine",
                      "timing": "HIP graph replay of 40 layers"}
        # decode-size MoE (T tokens, each through its 8 experts): latency per call
        dec = {}
        for Tq in (1, 4, 8):
            xq = torch.from_numpy(F.synth_activations(Tq, E, seed=50 + Tq)).to(dev)
            aqq, ascq, _ = qm.quantize_act(xq, M_stride=16)
            lgq = torch.from_numpy(F.zipf_router_logits(Tq, NE, seed=60 + Tq)).to(dev)
            wsq = qm.moe_workspace(Tq, NE, NU, E, Fd, device=dev)
            xoq = torch.empty((Tq, E), device=dev)
            msq = timed_graph(lambda i: qm.moe_grouped(ws_[0], ws_[1], ws_[2], NE, lgq, NU, aqq, ascq, xoq, wsq),
                              args, stream)
            ebytes = Tq * NU * 3 * F.weight_bytes(F.IQ4_XS, Fd, E)  # (upper bound: distinct experts x 3 matrices)
            dec[str(Tq)] = {"us_per_call": round(msq * 1e3, 1), "expert_bytes_upper_bound": ebytes}
        out["moe"]["decode"] = dec
        for w_ in ws_:
            w_.release()

    # ---------------- the other BASELINE configs and the activation producers (reported)
    if args.only in ("all", "report"):
        rep = {}
        for name, qtype, N, K, seed in (("q8_0_gemv_4096x4096", F.Q8_0, 4096, 4096, 0),
                                         ("iq3_s_gemv_5120x5120", F.IQ3_S, 5120, 5120, 3)):
            W = F.synth_weight(qtype, N, K, seed=seed)
            Wd = torch.from_numpy(W).to(dev)
            # rotate more than the 256 MB Infinity Cache holds, so every launch reads its weight from HBM
            ncopy = 2 if args.profile else max(args.copies, -(-300_000_000 // F.weight_bytes(qtype, N, K)))
            copies = [qm.QWeight(qtype, Wd, N, K) for _ in range(ncopy)]
            del Wd
            x = torch.from_numpy(F.synth_activations(1, K, seed=seed)).to(dev)
            aq, asc, absum = qm.quantize_act(x, M_stride=16)
            C = torch.empty((1, N), device=dev)
            msg = timed_graph(lambda i, copies=copies, aq=aq, asc=asc, absum=absum, C=C, N=N:
                              qm.gemv(copies[i % len(copies)], aq, asc, absum, C=C, ldc=N), args, stream)
            b = F.weight_bytes(qtype, N, K)
            rep[name] = {"us_per_launch": round(msg * 1e3, 2), "weight_GB/s": round(b / (msg * 1e-3) / 1e9, 1),
                         "frac_of_hbm_peak": round(b / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "weight_bytes": b,
                         "rotation": f"{ncopy} copies x {b} B = {ncopy * b / 1e6:.0f} MB"}
            if qtype == F.IQ3_S:
                M = 512
                xm = torch.from_numpy(F.synth_activations(M, K, seed=seed)).to(dev)
                aqm, ascm, absm = qm.quantize_act(xm)
                Cm = torch.empty((M, N), device=dev)
                msm, _ = timed(lambda i: qm.gemm(copies[0], aqm, ascm, absm, C=Cm, ldc=N), max(2, args.steps // 5),
                               args.warmup, stream)
                ops = 2.0 * M * N * K
                rep["iq3_s_gemm_512x5120x5120"] = {"ms_per_launch": round(msm, 4),
                                                    "TOPS": round(ops / (msm * 1e-3) / 1e12, 1),
                                                    "frac_of_int8_peak": round(ops / (msm * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                                                    "ops": int(ops)}
            for c in copies:
                c.release()
        # producers: decode (1 row) and prompt (2048 rows) sizes of the 27B-class shapes; bytes = f32 inputs read +
        # int8 rows, per-32 scales and per-16 sums written (+ the residual written back for add_norm_quant)
        K, Fd = 5120, 17408
        prod = {}
        for M in (1, 2048):
            x = torch.randn((M, K), device=dev)
            wv = torch.randn((K,), device=dev)
            gu = torch.randn((M, 2 * Fd), device=dev)
            t = torch.randn((M, K), device=dev)
            outb = lambda n: n + n // 32 * 4 + n // 16 * 2
            cases = (("rmsnorm_quant", lambda i: qm.rmsnorm_quant(x, wv, 1e-6), M * (4 * K) + 4 * K + M * outb(K)),
                     ("swiglu_quant", lambda i: qm.swiglu_quant(gu, Fd, fused=True), M * 8 * Fd + M * outb(Fd)),
                     ("add_norm_quant", lambda i: qm.add_norm_quant(x, t, wv, 1e-6, 1.0),
                      M * 12 * K + 4 * K + M * outb(K)))
            for nm, fn, byts in cases:
                # (both sizes as graph replays: an eager launch through the Python wrapper costs tens of microseconds of
                #  host time, more than the 2048-row kernels themselves; 20 launches per graph at 2048 rows)
                msp = timed_graph(fn, args, stream) if M == 1 else timed_graph_n(fn, 20, stream)
                prod[f"{nm}_M{M}"] = {"us": round(msp * 1e3, 2), "GB/s": round(byts / (msp * 1e-3) / 1e9, 1)}
        rep["producers_K5120_F17408"] = prod
        if not args.profile:
            # every weight type at the gate/up shape (K 5120 -> N 17408, batch 1), rotated over more than 256 MB
            K, N = 5120, 17408
            x = torch.from_numpy(F.synth_activations(1, K, seed=70)).to(dev)
            aq, asc, absum = qm.quantize_act(x, M_stride=16)
            C = torch.empty((1, N), device=dev)
            types = {}
            for qtype in sorted(F.TYPE_NAMES):
                Wd = torch.from_numpy(F.synth_weight(qtype, N, K, seed=71)).to(dev)
                b = F.weight_bytes(qtype, N, K)
                ncopy = max(2, -(-300_000_000 // b))
                copies = [qm.QWeight(qtype, Wd, N, K) for _ in range(ncopy)]
                del Wd
                msg = timed_graph(lambda i, copies=copies: qm.gemv(copies[i % len(copies)], aq, asc, absum, C=C, ldc=N),
                                  args, stream)
                types[F.TYPE_NAMES[qtype]] = {"us_per_launch": round(msg * 1e3, 2),
                                              "weight_GB/s": round(b / (msg * 1e-3) / 1e9, 1),
                                              "frac_of_hbm_peak": round(b / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                              "copies": ncopy}
                for c in copies:
                    c.release()
            rep["gemv_types_5120x17408"] = types
        out["reported"] = rep
        torch.cuda.empty_cache()

    if args.profile:
        # calibration copy for the FETCH_SIZE / WRITE_SIZE counters: 1 GiB read + 1 GiB written
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev).fill_(1.0)
        b = torch.empty_like(a)
        for _ in range(2):
            b.copy_(a)
        torch.cuda.synchronize()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
