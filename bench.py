#!/usr/bin/env python3
"""Benchmark of the qvx engine on one MI355X, against the BASELINE.json metric:
"Q4_K GEMV HBM GB/s (% of peak) at M=1; Q4_K prefill GEMM TFLOPS (% MFMA)".

A step is one Q4_K GEMV 4096 -> 14336 at M=1 (gate/up shape) over one of
`--copies` distinct seeded weight copies (>= 1 GiB in total, so every timed read comes from HBM
rather than the 256 MB Infinity Cache).  `value` is algorithmic bytes per step (weights +
activation + output) / time per step, with inputs resident in HBM; the K steps are recorded once
into one HIP graph (a qvx_plan) and replayed, so the time is the device's, not the host's per-call
launch cost (the eager launch loop is timed too and reported beside it).  The prefill GEMM
(Q4_K 4096 -> 14336, fp16 X, M in {2048, 512, 128}; bf16 MFMA, fp16 MFMA and
int8 MFMA variants) is reported beside it, and so are every GEMV point of configs[0..2] and the
config-5 decode sweep.  `cpu_baseline` times the reference's own CPU qmatmul
(oracle/_ref, built from the reference's sources) on the same weights on this host's cores.
`roofline.traffic` comes from the committed rocprofv3 PMC summary of this same GEMV
(profiles/q4k_gemv_4096x14336_m1.traffic.json: FETCH_SIZE / WRITE_SIZE per dispatch, each scaled
by the counter's reading for a plain device copy of known size), or is null when that file is absent.

Prints exactly one JSON line on stdout; diagnostics go to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # MI355X dense bf16 / fp16 MFMA
ROWS, COLS = 14336, 4096       # Q4_K gate/up projection of Llama-3-8B
Q4K_ROW_BYTES = COLS // 256 * 144
GEMV_KERNEL = "qvx::k_gemv_mx<1, 2, 1, 0>"   # matrix-core Q4_K GEMV, one vector per launch, no fused epilogue
GEMM_KERNEL = "qvx::k_qgemm_q4kq<0, 256> + qvx::k_qgemm_q4k<0, 192>"  # bf16, the two launches of the M=2048 plan
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4k_gemv_4096x14336_m1.traffic.json")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(rows, cols, m, wbytes):
    return wbytes + 4 * m * cols + 4 * m * rows


def cpu_baseline(w_host, x_host, rows, cols, budget_s=10.0):
    """The reference's CPU qmatmul (oracle/_ref, else the C restatement) on this host's cores."""
    import numpy as np
    import oracle
    kind, fn = "reference", None
    so = oracle.ref_lib()
    if so is not None:
        fn = so.qvxr_qmatmul
        dot = so.qvxr_dot_kernel().decode()
    else:
        kind = "port"
        so = oracle.lib()
        fn = so.qvxo_qmatmul
        dot = so.qvxo_dot_kernel().decode()
    out = np.zeros(rows, np.float32)
    wp = w_host.ctypes.data
    fn(out, wp, 12, x_host, rows, cols)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 50000):
        t0 = time.perf_counter()
        fn(out, wp, 12, x_host, rows, cols)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    nbytes = algorithmic_bytes(rows, cols, 1, w_host.size)
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": kind,
        "sample": f"Q4_K GEMV {cols}->{rows} M=1, same seeded blocks, 1 warm-up + median of {len(times)} runs "
                  f"({sum(times):.1f} s), OpenMP threads={cores}, dot kernel={dot}",
        "ms_per_gemv": round(med * 1e3, 3),
    }


def cpu_operator():
    """(kind, qmatmul_n function, dot kernel name, threads): the reference's own CPU qmatmulN
    (oracle/_ref, built from the reference's sources), else the C restatement."""
    import oracle
    so = oracle.ref_lib()
    if so is not None:
        kind, fn, dot = "reference", so.qvxr_qmatmul_n, so.qvxr_dot_kernel().decode()
    else:
        so = oracle.lib()
        kind, fn, dot = "port", so.qvxo_qmatmul_n, so.qvxo_dot_kernel().decode()
    cores = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
    return kind, fn, dot, cores


def cpu_time(fn, w_host, t, X_host, m, rows, cols, budget_s=0.6):
    """Median seconds of the CPU operator over >= 5 runs after one warm-up (steady clock), up to
    about budget_s of work."""
    import numpy as np
    out = np.zeros((m, rows), np.float32)
    wp = w_host.ctypes.data
    X = np.ascontiguousarray(X_host, np.float32)
    if not fn(out, wp, t, X, m, rows, cols):
        raise RuntimeError(f"CPU qmatmulN refused type {t}")
    times = []
    t_end = time.perf_counter() + budget_s
    while len(times) < 5 or (time.perf_counter() < t_end and len(times) < 200):
        t0 = time.perf_counter()
        fn(out, wp, t, X, m, rows, cols)
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


# BASELINE configs[0..2] GEMV points: (name, ggml type, rows, cols, M values, scale multiplier)
CONFIG_GEMVS = (
    ("C1 Q8_0 4096x4096", 8, 4096, 4096, (1,), 0.01),
    ("C2 Q4_0 up 4096->11008", 2, 11008, 4096, (1,), 0.02),
    ("C2 Q4_0 down 11008->4096", 2, 4096, 11008, (1,), 0.02),
    ("C3 Q4_K gate/up 4096->14336", 12, 14336, 4096, (1, 4, 16), 1e-3),
    ("C3 Q4_K down 14336->4096", 12, 4096, 14336, (1, 4, 16), 1e-3),
    ("C3 Q6_K lm_head 4096->128256", 14, 128256, 4096, (1, 4, 16), 1e-3),
)


def config_gemvs(torch, stream, steps, cpu=True):
    """Every GEMV point of BASELINE configs[0..2]: enough seeded weight copies (>= 1 GiB) cycled so
    each launch reads HBM; n qmatmul_n calls recorded into one HIP graph (a qvx_plan), replayed,
    and timed with HIP events (the device's time per call, not the host's per-call cost)."""
    import qorvix_amd as qvx
    from qorvix_amd import decode
    sh = stream.cuda_stream
    out = []
    for name, t, rows, cols, ms, mul in CONFIG_GEMVS:
        wb = qvx.weight_bytes(t, rows, cols)
        ncopy = max(2, -(-(1 << 30) // wb))
        ws = [decode.DevWeight(qvx.empty_weight(t, rows, cols), t, rows, cols) for _ in range(ncopy)]
        for i, w in enumerate(ws):
            qvx.fill_synthetic_t(w.data, t, rows, cols, seed=1000 + 17 * i + t, scale_mul=mul)
        for m in ms:
            X = torch.empty((m, cols), dtype=torch.float32, device="cuda")
            qvx.fill_normal_t(X, seed=77 + m)
            Y = torch.empty((m, rows), dtype=torch.float32, device="cuda")
            n = max(2 * ncopy, min(steps, int(2e-3 / max(wb / 4e12, 1e-6))))  # ~2 ms of work per point
            plan = decode.Plan()
            for i in range(n):
                plan.add(Y, ws[i % ncopy], X, m)
            plan.instantiate()
            plan.launch(sh)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            plan.launch(sh)
            plan.launch(sh)
            e1.record(stream)
            torch.cuda.synchronize()
            plan.close()
            us = e0.elapsed_time(e1) / (2 * n) * 1e3
            ab = algorithmic_bytes(rows, cols, m, wb)
            gbs = ab / (us * 1e-6) / 1e9
            rec = {"config": name, "M": m, "us": round(us, 2), "algorithmic_bytes": ab, "gb_s": round(gbs, 1),
                   "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "calls_timed": 2 * n, "weight_copies": ncopy}
            cpu_note = ""
            if cpu:  # the reference CPU operator on the same blocks and activations, this host's cores
                kind, fn, dot, cores = cpu_operator()
                sec, runs = cpu_time(fn, ws[0].data.cpu().numpy(), t, X.cpu().numpy(), m, rows, cols)
                rec["cpu"] = {"kind": kind, "us": round(sec * 1e6, 1), "gb_s": round(ab / sec / 1e9, 2), "runs": runs,
                              "threads": cores, "dot_kernel": dot}
                cpu_note = f"; CPU {kind} {sec * 1e3:.2f} ms ({ab / sec / 1e9:.1f} GB/s)"
            out.append(rec)
            log(f"[bench] {name} M={m}: {us:.2f} us, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)"
                + cpu_note)
            del X, Y
        del ws
        torch.cuda.empty_cache()
    return out


def decode_sweep(torch, stream, steps, cpu=True):
    """Config 5: the 225 GEMVs of one Llama-3-8B Q4_K_M token (32 layers x q, k, v, o, gate, up,
    down + the Q6_K LM head, 4.54 GiB of weights, cold in HBM every token) replayed as one HIP
    graph, at M = 1 and M = 8.  Rate = algorithmic bytes per token / time per token."""
    from qorvix_amd import decode
    model = decode.Model.synthetic(n_layers=decode.N_LAYERS, lm_head=True, seed=5)
    torch.cuda.synchronize()
    sh = stream.cuda_stream
    out = {"workload": "Llama-3-8B Q4_K_M decode weight sweep (BASELINE configs[4]): 32 x 7 projections "
                       "+ Q6_K lm_head = 225 GEMVs per token, one HIP graph per token, GEMVs in call order",
           "weight_bytes_per_token": model.nbytes}
    def time_step(mdl, m, concurrent, ops=None):
        if ops == "grouped":
            st = decode.DecodeStep(mdl, m, grouped=True)
        elif ops == "fused_grouped":
            st = decode.FusedDecodeStep(mdl, m, grouped=True)
        elif ops == "fused":
            st = decode.FusedDecodeStep(mdl, m)
        elif ops == "separate":
            st = decode.OpsDecodeStep(mdl, m)
            with torch.cuda.stream(stream):
                st.capture()
        else:
            st = decode.DecodeStep(mdl, m, concurrent=concurrent)
        with torch.cuda.stream(stream):
            for _ in range(3):
                st.replay(sh)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                st.replay(sh)
            e1.record(stream)
        torch.cuda.synchronize()
        if ops != "separate":
            st.plan.close()
        return e0.elapsed_time(e1) / steps

    fused = model.fused()  # q|k and gate|up stacked: 5 GEMVs a layer
    fops = model.fused_ops()  # ... and the RMSNorms and the SwiGLU folded in (gate|up interleaved)
    for m in (1, 8):
        ms = time_step(model, m, False)
        ms_br = time_step(model, m, True)
        ms_fu = time_step(fused, m, False)
        ms_ops = time_step(fops, m, False, ops="fused")
        ms_sep = time_step(model, m, False, ops="separate")
        ms_gr = time_step(model, m, False, ops="grouped") if m == 1 else None
        ms_fgr = time_step(fused, m, False, ops="grouped") if m == 1 else None
        ms_ogr = time_step(fops, m, False, ops="fused_grouped") if m == 1 else None
        _, ab = decode.sweep_bytes(m)
        gbs = ab / (ms * 1e-3) / 1e9
        out[f"M{m}"] = {"ms_per_token": round(ms, 4), "algorithmic_bytes_per_token": ab, "gb_s": round(gbs, 1),
                        "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "tokens_timed": steps,
                        "ms_per_token_qkv_gateup_branches": round(ms_br, 4),
                        "ms_per_token_fused_qk_gateup": round(ms_fu, 4),
                        "gb_s_fused_qk_gateup": round(ab / (ms_fu * 1e-3) / 1e9, 1),
                        "ms_per_token_fused_ops": round(ms_ops, 4),
                        "gb_s_fused_ops": round(ab / (ms_ops * 1e-3) / 1e9, 1),
                        "ms_per_token_separate_ops": round(ms_sep, 4),
                        **({"ms_per_token_grouped_qkv_gateup": round(ms_gr, 4),
                            "gb_s_grouped_qkv_gateup": round(ab / (ms_gr * 1e-3) / 1e9, 1),
                            "ms_per_token_grouped_qk_v": round(ms_fgr, 4),
                            "gb_s_grouped_qk_v": round(ab / (ms_fgr * 1e-3) / 1e9, 1),
                            "ms_per_token_fused_ops_grouped": round(ms_ogr, 4),
                            "gb_s_fused_ops_grouped": round(ab / (ms_ogr * 1e-3) / 1e9, 1),
                            "grouped_note": "grouped_qkv_gateup: q, k, v (Q6_K) in one grouped launch and gate, "
                                            "up in another (qvx_qmatmul_group, 4 launches a layer); grouped_qk_v: "
                                            "q|k stacked grouped with v, gate|up stacked (4 launches a layer); "
                                            "fused_ops_grouped: the fused ops with q|k and v on the normed state "
                                            "in one grouped launch (4 launches a layer)"}
                           if ms_gr else {}),
                        "fused_ops_note": "q|k and v with the attention RMSNorm folded in, o, gate|up with the FFN "
                                          "RMSNorm and the SwiGLU epilogue, down on that SwiGLU output, LM head with "
                                          "the output norm: 5 launches a layer + 1 (161 a token); separate_ops: the "
                                          "reference's op sequence, one launch per op (2 RMSNorms, 7 GEMVs, 1 SwiGLU a "
                                          "layer + norm and LM head = 322 a token), one graph"}
        log(f"[bench] sweep M={m}: {ms:.3f} ms/token, {gbs:.0f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak); "
            f"{ms_br:.3f} ms/token with q/k/v and gate/up as concurrent graph branches; {ms_fu:.3f} ms/token with "
            f"q|k and gate|up stacked (5 GEMVs a layer); {ms_ops:.3f} ms/token with the norms and SwiGLU folded in "
            f"(the same ops as separate launches: {ms_sep:.3f})"
            + (f"; {ms_gr:.3f} ms/token with q/k/v and gate/up as grouped launches, {ms_fgr:.3f} with q|k stacked "
               f"and grouped with v, {ms_ogr:.3f} fused ops with q|k and v grouped (4 launches a layer)"
               if ms_gr else ""))
        if cpu:
            # the reference CPU operator on layer 0's seven projections and the LM head (same blocks,
            # seeded activations); per token = 32 x layer + LM head
            import numpy as np
            kind, fn, dot, cores = cpu_operator()
            rng = np.random.default_rng(5 + m)
            layer_s = 0.0
            for name, rows, cols, t, _ in decode.LAYER_SPECS:
                w = model.layers[0][name]
                sec, _ = cpu_time(fn, w.data.cpu().numpy(), t, rng.standard_normal((m, cols)), m, rows, cols, 0.2)
                layer_s += sec
            lm = model.lm_head
            lm_s, _ = cpu_time(fn, lm.data.cpu().numpy(), lm.type, rng.standard_normal((m, lm.cols)), m, lm.rows,
                               lm.cols, 0.2)
            cpu_ms = (decode.N_LAYERS * layer_s + lm_s) * 1e3
            out[f"M{m}"]["cpu"] = {"kind": kind, "ms_per_token": round(cpu_ms, 2),
                                   "gb_s": round(ab / (cpu_ms * 1e-3) / 1e9, 2), "threads": cores, "dot_kernel": dot,
                                   "sample": "layer 0's 7 projections and the LM head, median of >= 5 runs each; "
                                             "per token = 32 x layer + LM head"}
            log(f"[bench] sweep M={m} CPU {kind}: {cpu_ms:.1f} ms/token ({ab / (cpu_ms * 1e-3) / 1e9:.1f} GB/s)")
    # Prefill: M prompt positions through every projection as one GEMM each (qvx_qgemm_f16, fp16 X;
    # Q4_K and Q6_K on the hand-written raw-block MFMA kernels) and the LM head
    # on the last position.  The reference prefills token by token (generator.cpp:24-28), one decode
    # step per position: its equivalent here is M x the M = 1 sweep time.
    def time_prefill(mdl, mp, reps=3):
        st = decode.PrefillStep(mdl, mp)
        st.run(sh)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            st.run(sh)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps, st.flops()

    def time_prefill_graph(mdl, mp, reps=3):
        # the same step captured into one graph (every GEMM through the no-allocation entry point)
        st = decode.PrefillStep(mdl, mp)
        st.capture()
        cur = torch.cuda.current_stream()
        st.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(cur)
        for _ in range(reps):
            st.replay()
        e1.record(cur)
        torch.cuda.synchronize()
        del st
        return e0.elapsed_time(e1) / reps

    pre = {}
    for mp in (512, 2048):
        ms, flops = time_prefill(model, mp)
        ms_fu, _ = time_prefill(fused, mp)
        ms_g = time_prefill_graph(model, mp)
        ms_gfu = time_prefill_graph(fused, mp)
        tf = flops / (ms * 1e-3) / 1e12
        tbt = mp * out["M1"]["ms_per_token"]
        pre[f"M{mp}"] = {"ms": round(ms, 3), "tokens_per_s": round(mp / (ms * 1e-3), 1), "tflops": round(tf, 1),
                         "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4), "runs_timed": 3,
                         "token_by_token_ms": round(tbt, 2), "speedup_vs_token_by_token": round(tbt / ms, 1),
                         "ms_fused_qk_gateup": round(ms_fu, 3),
                         "tokens_per_s_fused_qk_gateup": round(mp / (ms_fu * 1e-3), 1),
                         "ms_graph": round(ms_g, 3), "tokens_per_s_graph": round(mp / (ms_g * 1e-3), 1),
                         "tflops_graph": round(flops / (ms_g * 1e-3) / 1e12, 1),
                         "ms_graph_fused_qk_gateup": round(ms_gfu, 3),
                         "graph_note": "the step captured into one HIP graph (qvx_qgemm_f16_noalloc), "
                                       "replayed: no host launch gaps"}
        log(f"[bench] prefill M={mp}: {ms:.2f} ms ({mp / (ms * 1e-3):.0f} tokens/s, {tf:.0f} TFLOP/s); token by token "
            f"{tbt:.1f} ms; {ms_fu:.2f} ms with q|k and gate|up stacked; as one graph {ms_g:.2f} ms "
            f"({mp / (ms_g * 1e-3):.0f} tokens/s), stacked {ms_gfu:.2f} ms")
    out["prefill"] = {"workload": "Llama-3-8B Q4_K_M prompt prefill: 32 x 7 projections as GEMMs over M positions "
                                  "(fp16 activations) + the Q6_K LM head on the last position", **pre}
    del model, fused, fops
    torch.cuda.empty_cache()
    return out


def hbm_context(torch, stream, copies):
    """Measured HBM rates beside the assumed peak, for context: the engine's bare streaming read
    (qvx_bench_read, one 16-byte load per thread) over the GEMV's own weight copies (same bytes, same
    cycling past the Infinity Cache, replayed as one graph like the GEMV leg) -- the most one launch
    of that size reads -- and over 1 GiB; and a 512 MiB device-to-device copy (read + write bytes)."""
    import qorvix_amd as qvx
    so = qvx.lib()
    sh = stream.cuda_stream
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")

    def read(buf, nbytes):
        qvx._check(so.qvx_bench_read(buf.data_ptr(), nbytes, flag.data_ptr(), torch.cuda.current_stream().cuda_stream),
                   "qvx_bench_read")

    nb = copies[0].numel()
    for c in copies:
        read(c, nb)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for c in copies:
            read(c, nb)
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    us_small = e0.elapsed_time(e1) * 1e3 / (reps * len(copies))
    del g

    def timed(fn, n=5):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(n):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            torch.cuda.synchronize()
            ts.append(a.elapsed_time(b) * 1e-3)
        return sorted(ts)[len(ts) // 2]
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    big.fill_(7)
    with torch.cuda.stream(stream):
        t_big = timed(lambda: read(big, 1 << 30))
    del big
    src = torch.empty(512 << 20, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    with torch.cuda.stream(stream):
        t_copy = timed(lambda: dst.copy_(src))
    del src, dst
    torch.cuda.empty_cache()
    assert int(flag.item()) == 0  # no word matched the pattern: nothing was stored
    return {"read_us_gemv_weight_bytes": round(us_small, 2), "read_gbs_gemv_weight_bytes": round(nb / us_small / 1e3, 1),
            "read_gbs_1gib": round((1 << 30) / t_big / 1e9, 1),
            "copy_gbs_512mib": round(2 * (512 << 20) / t_copy / 1e9, 1),
            "peak_assumed_gbs": HBM_PEAK_GBS,
            "note": "qvx_bench_read (one 16-byte load per thread) over the GEMV's weight bytes cycled over its "
                    "weight copies (graph-timed), and over 1 GiB; device copy of 512 MiB counts read + write "
                    "bytes; context for the GEMV's HBM fraction, not part of the metric"}


def dequant_leg(torch, stream, t, copies, reps=20):
    """qvx_dequantize (the reference's dequantize) of one Q4_K 4096 -> 14336 weight to fp32, cycling
    the weight copies, HIP events on the launch stream; bytes = block bytes read + 4 B written per
    element."""
    import qorvix_amd as qvx
    lib, sh = qvx.lib(), stream.cuda_stream
    n = ROWS * COLS
    out = torch.empty(n, dtype=torch.float32, device=stream.device)

    def d(i):
        rc = lib.qvx_dequantize(t, copies[i % len(copies)].data_ptr(), out.data_ptr(), n, sh)
        if rc != 0:
            raise RuntimeError(f"qvx_dequantize failed: {qvx.strerror(rc)}")
    for i in range(3):
        d(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        d(i)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    nbytes = copies[0].numel() + 4 * n
    gbs = nbytes / (us * 1e-6) / 1e9
    log(f"[bench] dequantize Q4_K {ROWS}x{COLS} -> fp32: {us:.1f} us, {gbs:.0f} GB/s "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    del out
    return {"workload": f"qvx_dequantize Q4_K {ROWS}x{COLS} -> fp32", "us": round(us, 2), "bytes": nbytes,
            "gbs": round(gbs, 1), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def gemm_leg(torch, stream, t, wps, copies, steps, cpu):
    """Q4_K 4096 -> 14336 prefill GEMM at M = 2048, 512, 128 in the bf16, fp16 and
    int8 variants, each call timed whole (prepass + GEMM) with HIP events on the launch stream, and the
    reference CPU qmatmulN beside it on a 64-token sample; then the Q6_K ffn_down GEMM (the Q6_K tensor
    of a Q4_K_M layer) at M = 2048."""
    import qorvix_amd as qvx
    lib, sh, dev = qvx.lib(), stream.cuda_stream, stream.device
    gemm = {}
    try:
        for M in (2048, 512, 128):
            X = torch.empty((M, COLS), dtype=torch.float16, device=dev)
            qvx.fill_normal_t(X, seed=11, mul=0.5)
            Y = torch.empty((M, ROWS), dtype=torch.float32, device=dev)
            for name, var in (("bf16", qvx.GEMM_BF16), ("f16", qvx.GEMM_F16), ("i8", qvx.GEMM_I8)):
                def g(i):
                    rc = lib.qvx_qgemm_f16(Y.data_ptr(), wps[i % len(wps)], t, X.data_ptr(), M, ROWS, COLS, var, sh)
                    if rc != 0:
                        raise RuntimeError(f"qvx_qgemm_f16 failed: {qvx.strerror(rc)}")
                for i in range(10):  # warm-up; also lets the clock settle when this leg runs first
                    g(i)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(steps):
                    g(i)
                e1.record(stream)
                torch.cuda.synchronize()
                ms = e0.elapsed_time(e1) / steps
                tflops = 2.0 * M * ROWS * COLS / (ms * 1e-3) / 1e12
                gemm[f"{name}_M{M}"] = {"ms": round(ms, 4), "tflops": round(tflops, 1),
                                        "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4)}
                log(f"[bench] GEMM {name} M={M}: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s "
                    f"({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")
            if cpu:
                # the reference CPU qmatmulN on the first 64 tokens of X (fp16 -> fp32 exactly; 64 is
                # the operator's own vector tile), same blocks; GFLOP/s extrapolates per token
                kind, fn, dot, cores = cpu_operator()
                ms_tok = 64
                Xs = X[:ms_tok].float().cpu().numpy()
                sec, runs = cpu_time(fn, copies[0].cpu().numpy(), t, Xs, ms_tok, ROWS, COLS)
                gf = 2.0 * ms_tok * ROWS * COLS / sec / 1e9
                gemm[f"cpu_M{M}"] = {"kind": kind, "gflops": round(gf, 1), "ms_for_sample": round(sec * 1e3, 2),
                                     "ms_extrapolated": round(sec * 1e3 * M / ms_tok, 1), "runs": runs,
                                     "threads": cores, "dot_kernel": dot,
                                     "sample": f"first {ms_tok} of the {M} tokens (qmatmulN, X converted fp16->fp32)"}
                log(f"[bench] GEMM M={M} CPU {kind}: {gf:.1f} GFLOP/s on a {ms_tok}-token sample")
            del X, Y
        # the Q6_K prefill GEMM on Llama-3-8B's ffn_down (14336 -> 4096, the Q6_K tensor of a Q4_K_M
        # layer), M = 2048, fp16 MFMA: four seeded weight copies cycled, each call timed whole
        q6, q6r, q6c, q6m = qvx.Q6_K, 4096, 14336, 2048
        w6 = [qvx.empty_weight(q6, q6r, q6c, dev) for _ in range(4)]
        for i, w in enumerate(w6):
            qvx.fill_synthetic_t(w, q6, q6r, q6c, seed=300 + i, scale_mul=1e-3)
        X = torch.empty((q6m, q6c), dtype=torch.float16, device=dev)
        qvx.fill_normal_t(X, seed=13, mul=0.5)
        Y = torch.empty((q6m, q6r), dtype=torch.float32, device=dev)
        def g6(i):
            rc = lib.qvx_qgemm_f16(Y.data_ptr(), w6[i % 4].data_ptr(), q6, X.data_ptr(), q6m, q6r, q6c, qvx.GEMM_F16, sh)
            if rc != 0:
                raise RuntimeError(f"qvx_qgemm_f16 (Q6_K) failed: {qvx.strerror(rc)}")
        for i in range(10):
            g6(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            g6(i)
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        tflops = 2.0 * q6m * q6r * q6c / (ms * 1e-3) / 1e12
        gemm["q6k_ffn_down_f16_M2048"] = {"ms": round(ms, 4), "tflops": round(tflops, 1),
                                           "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
                                           "shape": "Q6_K 14336->4096 (ffn_down), M=2048, fp16 MFMA"}
        log(f"[bench] GEMM Q6_K ffn_down f16 M=2048: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s "
            f"({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")
        del X, Y, w6
        # the other on-path formats' prefill GEMM (BASELINE configs[0..1] weights at M = 2048, bf16):
        # 16-bit dequantisation of the weight, then the plain matrix-core GEMM, timed together
        for name, tq, r, c in (("Q8_0 4096x4096", qvx.Q8_0, 4096, 4096), ("Q4_0 up 4096->11008", qvx.Q4_0, 11008, 4096),
                               ("Q4_0 down 11008->4096", qvx.Q4_0, 4096, 11008)):
            M = 2048
            wq = [qvx.empty_weight(tq, r, c, dev) for _ in range(4)]
            for i, w in enumerate(wq):
                qvx.fill_synthetic_t(w, tq, r, c, seed=400 + i, scale_mul=1e-3)
            X = torch.empty((M, c), dtype=torch.float16, device=dev)
            qvx.fill_normal_t(X, seed=14, mul=0.5)
            Y = torch.empty((M, r), dtype=torch.float32, device=dev)
            def gq(i):
                rc = lib.qvx_qgemm_f16(Y.data_ptr(), wq[i % 4].data_ptr(), tq, X.data_ptr(), M, r, c, qvx.GEMM_BF16, sh)
                if rc != 0:
                    raise RuntimeError(f"qvx_qgemm_f16 ({name}) failed: {qvx.strerror(rc)}")
            for i in range(10):
                gq(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(steps):
                gq(i)
            e1.record(stream)
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
            tflops = 2.0 * M * r * c / (ms * 1e-3) / 1e12
            gemm[f"{name.split()[0].lower()}_{r}x{c}_bf16_M2048"] = {
                "ms": round(ms, 4), "tflops": round(tflops, 1), "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
                "shape": f"{name}, M=2048, bf16 MFMA (16-bit dequantisation + plain GEMM, one call)"}
            log(f"[bench] GEMM {name} bf16 M=2048: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s "
                f"({100 * tflops / BF16_PEAK_TFLOPS:.1f}% of bf16 peak)")
            del X, Y, wq
    except RuntimeError as e:  # report, never hide: the JSON carries the error
        gemm["error"] = str(e)
        log(f"[bench] GEMM failed: {e}")
    return gemm


def qmatmul_n_leg(torch, stream, steps, cpu):
    """qvx_qmatmul_n at encoder batch sizes (the reference's qmatmulN / wmatmulNBias callers, BERT /
    CLIP / Whisper encoders at nVec 256-577): Q4_K 4096 -> 14336 with fp32 X at M = 16, 64 and 512,
    every output bit-identical to the one-vector call.  Four seeded weight copies cycled, direct calls
    timed with HIP events on the launch stream; the reference CPU qmatmulN beside it on 64 vectors."""
    import qorvix_amd as qvx
    lib, sh, dev = qvx.lib(), stream.cuda_stream, stream.device
    t = qvx.Q4_K
    out = {"workload": "qvx_qmatmul_n, Q4_K 4096->14336, fp32 X [M,4096], fp32 out (activations converted "
                       "once, weights streamed once per 64 vectors)"}
    try:
        ws = [qvx.empty_weight(t, ROWS, COLS, dev) for _ in range(4)]
        for i, w in enumerate(ws):
            qvx.fill_synthetic_t(w, t, ROWS, COLS, seed=500 + i, scale_mul=1e-3)
        for M in (16, 64, 512):
            X = torch.empty((M, COLS), dtype=torch.float32, device=dev)
            qvx.fill_normal_t(X, seed=15)
            Y = torch.empty((M, ROWS), dtype=torch.float32, device=dev)
            def q(i):
                rc = lib.qvx_qmatmul_n(Y.data_ptr(), ws[i % 4].data_ptr(), t, X.data_ptr(), M, ROWS, COLS, sh)
                if rc != 0:
                    raise RuntimeError(f"qvx_qmatmul_n failed: {qvx.strerror(rc)}")
            for i in range(10):
                q(i)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(steps):
                q(i)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / steps * 1e3
            tops = 2.0 * M * ROWS * COLS / (us * 1e-6) / 1e12
            rec = {"us": round(us, 2), "effective_tops": round(tops, 1), "us_per_vector": round(us / M, 3)}
            note = ""
            if cpu and M == 64:
                kind, fn, dot, cores = cpu_operator()
                sec, runs = cpu_time(fn, ws[0].cpu().numpy(), t, X.cpu().numpy(), M, ROWS, COLS)
                rec["cpu"] = {"kind": kind, "us": round(sec * 1e6, 1), "runs": runs, "threads": cores, "dot_kernel": dot}
                note = f"; CPU {kind} {sec * 1e3:.2f} ms"
            out[f"M{M}"] = rec
            log(f"[bench] qmatmul_n Q4_K 4096->14336 M={M}: {us:.1f} us ({us / M:.2f} us/vector, "
                f"{tops:.1f} effective TOP/s){note}")
            del X, Y
        del ws
    except RuntimeError as e:  # report, never hide
        out["error"] = str(e)
        log(f"[bench] qmatmul_n failed: {e}")
    return out


def calibration_copy(torch, dev, mib):
    """One plain device copy of `mib` MiB: the PMC byte counters' scale for a known transfer."""
    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=dev)
    b = torch.empty(n, dtype=torch.uint8, device=dev)
    a.fill_(1)
    torch.cuda.synchronize()
    b.copy_(a)
    torch.cuda.synchronize()
    log(f"[bench] calibration copy of {mib} MiB done")
    del a, b


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=40)
    ap.add_argument("--copies", type=int, default=40, help="distinct weight copies cycled per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--gemm-steps", type=int, default=20)
    ap.add_argument("--gemv-only", action="store_true", help="only the GEMV leg (for profiler passes)")
    ap.add_argument("--sweep-steps", type=int, default=20, help="timed tokens of the config-5 decode sweep")
    ap.add_argument("--sweep-only", action="store_true", help="only the config-5 decode sweep (profiler passes)")
    ap.add_argument("--configs-only", action="store_true", help="only the configs[0..2] GEMV points (profiler passes)")
    ap.add_argument("--gemm-only", action="store_true", help="only the prefill GEMM leg (profiler passes)")
    ap.add_argument("--dequant-only", action="store_true", help="only the fp32 dequantisation leg (profiler passes)")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MiB",
                    help="also run one plain device copy of this many MiB (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the qvx engine has no multi-GPU "
              "path in this build.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import qorvix_amd as qvx

    assert torch.cuda.is_available(), "no GPU visible"
    qvx.lib()  # fails loudly if libqvx.so was not built
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    if args.sweep_only:  # profiler pass over the decode sweep alone
        print(json.dumps({"sweep": decode_sweep(torch, stream, args.sweep_steps, cpu=not args.no_cpu)}), flush=True)
        return
    if args.configs_only:  # profiler pass over the configs[0..2] GEMV points alone
        if args.calibrate_copy:
            calibration_copy(torch, dev, args.calibrate_copy)
        print(json.dumps({"config_gemvs": config_gemvs(torch, stream, 200, cpu=not args.no_cpu)}), flush=True)
        return
    t = qvx.Q4_K
    wbytes = qvx.weight_bytes(t, ROWS, COLS)

    # ---- data: seeded synthetic Q4_K blocks and x ~ N(0,1) ----------------
    copies = [qvx.empty_weight(t, ROWS, COLS, dev) for _ in range(args.copies)]
    for i, w in enumerate(copies):
        qvx.fill_synthetic_t(w, t, ROWS, COLS, seed=1000 + i, scale_mul=1e-3)
    x = torch.empty(COLS, dtype=torch.float32, device=dev)
    qvx.fill_normal_t(x, seed=7)
    out = torch.empty(ROWS, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    if args.dequant_only:  # profiler pass over the fp32 dequantisation leg alone
        if args.calibrate_copy:
            calibration_copy(torch, dev, args.calibrate_copy)
        print(json.dumps({"dequant": dequant_leg(torch, stream, t, copies)}), flush=True)
        return
    if args.gemm_only:  # profiler pass over the prefill GEMM leg alone
        wps = [w.data_ptr() for w in copies]
        print(json.dumps({"gemm": gemm_leg(torch, stream, t, wps, copies, args.gemm_steps, cpu=not args.no_cpu)}),
              flush=True)
        return
    log(f"[bench] {args.copies} Q4_K copies x {wbytes / 2**20:.1f} MiB = {args.copies * wbytes / 2**30:.2f} GiB")

    lib = qvx.lib()
    sh = stream.cuda_stream
    xp, op = x.data_ptr(), out.data_ptr()
    wps = [w.data_ptr() for w in copies]

    def step(i):
        rc = lib.qvx_qmatmul(op, wps[i % len(wps)], t, xp, ROWS, COLS, sh)
        if rc != 0:
            raise RuntimeError(f"qvx_qmatmul failed: {qvx.strerror(rc)}")

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()

    # ---- timed region: K steps between two events on the launch stream -------------------------
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(args.steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_total = ev0.elapsed_time(ev1)
    ms_eager = ms_total / args.steps
    nbytes = algorithmic_bytes(ROWS, COLS, 1, wbytes)
    log(f"[bench] GEMV eager: {args.steps} steps in {ms_total:.3f} ms (wall {wall * 1e3:.1f} ms): "
        f"{ms_eager * 1e3:.2f} us/step, {nbytes / (ms_eager * 1e-3) / 1e9:.0f} GB/s")

    # The same K steps recorded once into a qvx_plan (one HIP graph) and replayed: the device runs
    # the launches back to back whatever the host's per-call cost, which the eager loop above
    # includes when a launch takes longer to issue than the kernel takes to run.
    from qorvix_amd import decode
    plan = decode.Plan()
    for i in range(args.steps):
        plan.add(out, decode.DevWeight(copies[i % len(copies)], t, ROWS, COLS), x, 1)
    plan.instantiate()
    plan.launch(sh)
    torch.cuda.synchronize()
    reps = 3
    ev0.record(stream)
    for _ in range(reps):
        plan.launch(sh)
    ev1.record(stream)
    torch.cuda.synchronize()
    plan.close()
    ms_per_step = ev0.elapsed_time(ev1) / (reps * args.steps)
    gbs = nbytes / (ms_per_step * 1e-3) / 1e9
    log(f"[bench] GEMV graph: {reps} x {args.steps} steps: {ms_per_step * 1e3:.2f} us/step, {gbs:.0f} GB/s")

    # per-launch event pairs (kernel duration incl. event overhead), for the roofline line
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(64)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i + 7)
        b.record(stream)
    torch.cuda.synchronize()
    pair_us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)
    pair_med = statistics.median(pair_us)
    log(f"[bench] GEMV per-launch event pairs: median {pair_med:.2f} us, min {pair_us[0]:.2f} us")

    if args.calibrate_copy:
        calibration_copy(torch, dev, args.calibrate_copy)

    # ---- prefill GEMM ----------------------------------------------------
    gemm = {} if args.gemv_only else gemm_leg(torch, stream, t, wps, copies, args.gemm_steps, cpu=not args.no_cpu)
    deq = {}
    if not args.gemv_only:
        try:
            deq = dequant_leg(torch, stream, t, copies)
        except RuntimeError as e:  # report, never hide
            deq = {"error": str(e)}
            log(f"[bench] dequantize failed: {e}")

    # ---- qmatmul_n at encoder batch sizes ---------------------------------------------------------
    qn = {} if args.gemv_only else qmatmul_n_leg(torch, stream, args.gemm_steps, cpu=not args.no_cpu)

    # ---- every GEMV point of BASELINE configs[0..2] ----------------------------------------------
    cfgs = []
    if not args.gemv_only:
        try:
            cfgs = config_gemvs(torch, stream, 200, cpu=not args.no_cpu)
        except RuntimeError as e:  # report, never hide
            cfgs = [{"error": str(e)}]
            log(f"[bench] config GEMVs failed: {e}")

    # ---- full-model decode weight sweep ----------------------------------
    sweep = {}
    if not args.gemv_only:
        try:
            sweep = decode_sweep(torch, stream, args.sweep_steps, cpu=not args.no_cpu)
        except RuntimeError as e:  # report, never hide
            sweep = {"error": str(e)}
            log(f"[bench] sweep failed: {e}")

    # ---- CPU baseline (reference CPU operator on this host) ------------------------------------
    cpu = None
    if not args.no_cpu and not args.gemv_only:
        w_host = copies[0].cpu().numpy()
        x_host = x.cpu().numpy()
        cpu = cpu_baseline(w_host, x_host, ROWS, COLS)
        log(f"[bench] CPU baseline ({cpu['kind']}): {cpu['value']} GB/s, {cpu['ms_per_gemv']} ms/GEMV")

    hbm_ctx = hbm_context(torch, stream, copies)
    log(f"[bench] HBM context: bare read of the GEMV's {copies[0].numel()} weight bytes "
        f"{hbm_ctx['read_us_gemv_weight_bytes']} us ({hbm_ctx['read_gbs_gemv_weight_bytes']} GB/s), of 1 GiB "
        f"{hbm_ctx['read_gbs_1gib']} GB/s; device copy {hbm_ctx['copy_gbs_512mib']} GB/s (peak assumed "
        f"{HBM_PEAK_GBS:.0f} GB/s)")

    achieved = nbytes / (ms_per_step * 1e-3) / 1e9
    g2048 = gemm.get("bf16_M2048", {})
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    result = {
        "metric": "Q4_K GEMV HBM GB/s (% of peak) at M=1; Q4_K prefill GEMM TFLOPS (% MFMA)",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "ms_per_step_eager_loop": round(ms_eager, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "i8 MFMA, i32 accumulate, f32 fold",
        "arithmetic": "x rounded to 15-bit fixed point per 64-element group and split into two signed bytes; "
                      "Q4_K codes as int8; exact i32 dot products on v_mfma_i32_16x16x64_i8; each group's "
                      "scale/min fold and the sum over groups in fp32 (max-rel error vs exact <= 1e-3)",
        "data": "synthetic (seeded Q4_K blocks: fp16 d, dmin = |N(0,1)|*1e-3, uniform scale/quant bytes; x ~ N(0,1))",
        "config": {
            "workload": "Q4_K GEMV 4096->14336, M=1 (BASELINE configs[2]); one step = one GEMV",
            "rows": ROWS, "cols": COLS, "M": 1, "weight_copies": args.copies,
            "weight_bytes": wbytes, "algorithmic_bytes_per_step": nbytes,
        },
        "percent_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": GEMV_KERNEL,
            "per_launch_event_pair_us": round(pair_med, 3),
        },
        "isolated_call": {
            "note": "one GEMV between its own pair of events (launch ramp and drain not overlapped with a "
                    "neighbouring launch), median of 64",
            "us": round(pair_med, 3),
            "GB/s": round(nbytes / (pair_med * 1e-6) / 1e9, 1),
            "frac": round(nbytes / (pair_med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
        },
        "gemm": {
            "workload": "Q4_K 4096->14336 GEMM, X fp16 [M,4096], fp32 out (BASELINE configs[3])",
            "tflops_bf16_M2048": g2048.get("tflops"),
            "percent_of_bf16_peak_M2048": round(100 * g2048["frac_of_bf16_peak"], 2) if g2048 else None,
            "roofline": {
                "bound": "mfma",
                "achieved": g2048.get("tflops"),
                "peak": BF16_PEAK_TFLOPS,
                "unit": "TFLOP/s",
                "frac": g2048.get("frac_of_bf16_peak"),
                "traffic": None,
                "kernel": GEMM_KERNEL,
                "note": "one call = fp16->bf16 prepass + GEMM kernel, timed together; i8 rows count "
                        "2*M*N*K ops per call against the same bf16 peak",
            },
            "runs": gemm,
        },
        "config_gemvs": cfgs,
        "qmatmul_n": qn,
        "sweep": sweep,
        "cpu_baseline": cpu,
        "dequant": deq,
        "hbm_context": hbm_ctx,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
