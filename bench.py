"""Throughput of the packed-weight linear hot path on one MI355X.

Workload (the north-star shape): one SDXL-UNet
GEGLU-input linear 1280 -> 5120 on batch 2 x 1024 tokens (M = 2048), bf16,
winner optimizer flags (ratio-coherence gates, gf_consol = 50, no coh_pre),
fused dequant-GEMM mode.  One step = forward (dequant-GEMM) + backward
(dequant-GEMM dgrad, wgrad, v-hat EMA, packed update) + rebalance(), on
synthetic x ~ N(0,1) and dy ~ N(0, 1e-3), random-init weights.

Prints one JSON line.  value = dequant-matmul throughput of the whole step,
6 M N K / step time (TFLOP/s).  The step's entries are timed one by one (HIP
events around a HIP graph of back-to-back calls): forward, dgrad (main kernel
+ split reduction), wgrad with the v-hat partials and bias gradient in its
epilogue (+ the v-hat EMA kernels), packed update; bwd_products = the entry
the step's backward calls (dgrad, then the wgrad launch that also carries the
dgrad's split-K reduction, then the v-hat EMA).  roofline = the longest entry
the step calls against its roofline: a GEMM against dense bf16 MFMA peak at 2 M N K
algorithmic FLOP per product (4 M N K for bwd_products), the packed update against HBM peak at 10 algorithmic
B/param; rooflines = the same for every entry; traffic = HBM bytes per call
from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
(profiles/traffic_sdxl_1280x5120.txt) when present.  cpu_baseline = the same
step on the host: torch fp32 GEMMs + the CPU oracle's v-hat / update /
rebalance.

The step is timed from a HIP graph holding 5 consecutive steps (--graph-steps),
replayed back to back; every step's kernels run, only the replay launch is
shared by 5 steps.

`--only KERNEL` runs one entry of the step `--reps` times and exits (the
command the committed rocprofv3 summaries were taken with); KERNEL = fwd,
bwd, dgrad, wgrad, wgrad_vhat, vhat, update, materialize, or copy (a 256 MiB
device copy, the counter calibration).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

N_OUT, K_IN, M_TOK = 5120, 1280, 2048
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0
# VALU issue peak: 1024 SIMDs x 16 lanes per cycle at the 2.4 GHz peak engine
# clock (a wave64 VALU instruction holds a 16-lane SIMD for 4 cycles)
PEAK_VALU_TLANE_OPS = 1024 * 16 * 2.4e9 / 1e12
UPDATE_BYTES_PER_PARAM = 10      # int32 read + int32 write + bf16 grad read
DECODE_BYTES_PER_PARAM = 6       # int32 read + bf16 write


def _event_time_ms(fn, reps, torch):
    """Average GPU time of fn: `reps` calls captured back to back in one HIP
    graph, replayed and timed with events on the launching stream, so host
    launch overhead does not enter the figure."""
    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    n = 3
    e0.record()
    for _ in range(n):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (n * reps)


def _read_traffic():
    """HBM bytes per launch per kernel from the committed PMC summary:
    lines `kernel_key  fetch_bytes  write_bytes`."""
    path = os.path.join(ROOT, "profiles", "traffic_sdxl_1280x5120.txt")
    out = {}
    if not os.path.exists(path):
        return out
    for line in open(path):
        f = line.split()
        if len(f) == 3 and not line.startswith("#"):
            try:
                out[f[0]] = int(f[1]) + int(f[2])
            except ValueError:
                pass
    return out


def _read_valu_per_word():
    """VALU lane-instructions per packed word of the update kernel, from the
    committed PMC summary's line `valu_per_word apply_adamw X` (64 x
    SQ_INSTS_VALU / words)."""
    path = os.path.join(ROOT, "profiles", "pmc_sdxl_1280x5120.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "valu_per_word" and f[1] == "apply_adamw":
            try:
                return float(f[2])
            except ValueError:
                return None
    return None


def _cpu_model():
    """The host CPU's model name from /proc/cpuinfo (what lscpu prints)."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_leg(threads, max_s, max_steps):
    """Steps of the same workload on the host cores with `threads` threads:
    torch fp32 GEMMs and the CPU oracle's v-hat EMA, packed update and
    rebalance.  One untimed step, then steps until max_s seconds or
    max_steps steps."""
    import numpy as np
    import torch
    from oracle import oracle as O
    torch.set_num_threads(threads)
    O.set_threads(threads)
    rng = np.random.default_rng(0)
    x = torch.from_numpy(rng.standard_normal((M_TOK, K_IN)).astype(np.float32))
    dy = torch.from_numpy((rng.standard_normal((M_TOK, N_OUT)) * 1e-3).astype(np.float32))
    W0 = (rng.standard_normal((N_OUT, K_IN)) * (2.0 / (N_OUT + K_IN)) ** 0.5).astype(np.float32)
    pk, re, ce = O.load_weights(W0)
    vr = np.zeros(N_OUT, np.float32)
    vc = np.zeros(K_IN, np.float32)
    P = O.UpdateParams(alpha=0.1, beta1=0.0, weight_decay=0.0, step_cap=10.0, v_scale=0.0,
                       precond_p=0.5, gf_consol=50.0, drift_cancel_C=0.018036072144288578,
                       alpha_v_fast=0.001, wd_sv=0.0, wd_sf=0.0, gf_trust_delta_sq=1.0,
                       gate_gain=1.0, mantissa_bias=15)
    flags = (O.MASS_PRESERVE | O.APPLY_CHASE | O.TRACK_REBALANCE | O.GF_TRUST_REGION
             | O.GF_CONSOLIDATION | O.FIXED_COH | O.RATIO_COH)

    def step(salt):
        W = torch.from_numpy(O.bf16_bits_to_f32(O.materialize(pk, re, ce)).astype(np.float32))
        y = x @ W.T
        dx = dy @ W
        gw = dy.T @ x
        gb = O.f32_to_bf16_bits_array(gw.numpy())
        svi = O.vhat_ema(gb, vr, vc, 0.999)
        rm = np.zeros(N_OUT, np.int32)
        cm = np.zeros(K_IN, np.int32)
        S = O.UpdateScalars(lr=5e-4, eps=1e-10, chase_floor=0.9, leak_floor=0.999, v_bc=1.0,
                            salt=salt, consolidate=1)
        O.apply_adamw(pk, gb, None, re, ce, rm, cm, vr, vc, svi, None, P, S, flags)
        O.rebalance(pk, re, ce, rm, cm, seed=salt)
        return y, dx

    step(1)
    reps, t0 = 0, time.perf_counter()
    while True:
        step(2 + reps)
        reps += 1
        el = time.perf_counter() - t0
        if el > max_s or reps >= max_steps:
            break
    sec = el / reps
    return {"value": round(6.0 * M_TOK * N_OUT * K_IN / sec / 1e12, 4), "unit": "TFLOP/s", "cores": threads,
            "ms_per_step": round(sec * 1e3, 2), "steps_timed": reps}


def cpu_baseline():
    """The step on the GPU box's host cores, twice: with every CPU this
    process may run on (the reported value) and with one thread."""
    avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    full = cpu_baseline_leg(avail, 10.0, 10)
    one = cpu_baseline_leg(1, 12.0, 4)
    return dict(full, kind="port",
                sample=f"{full['steps_timed']} full steps of the 1280->5120 M=2048 workload on {avail} threads "
                       f"(and {one['steps_timed']} on 1 thread): torch fp32 GEMMs (fwd, dgrad, wgrad) + oracle "
                       "v-hat, update, rebalance",
                single_thread=one, os_cpu_count=os.cpu_count(), affinity_cpus=avail, cpu_model=_cpu_model(),
                omp_num_threads=os.environ.get("OMP_NUM_THREADS"))


def _graph_ms(step, warmup, steps, torch, per_graph=1):
    """Average time of one step replayed from a HIP graph of per_graph steps
    (events on the launching stream)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(per_graph):
            step()
    for _ in range(max(1, warmup // per_graph)):
        g.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // per_graph)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * per_graph)


# sum of (rows + columns) over config 4's 754 SDXL Linear and 1x1 weights: the
# watermark slab a GatedRebalance over the whole UNet reduces
CONFIG4_WATERMARKS = 2729216


def _next_rows(layer, xb, dy, gw, reps, warmup, steps, torch, ca, pb):
    """Context timings of the rows beside the step, on the same layer state:
    gradient noise (isotropic and Sigma_g), the prototype accumulate update
    (consf = 0), the coherence meter and the multi-layer watermark peak of the
    gated rebalance, and one training step of a 3 x 3 Concord conv."""
    from concord_amd import _lib as C
    dev = xb.device
    params = N_OUT * K_IN

    def hbm(t_ms, nbytes, kernel):
        a = nbytes / (t_ms * 1e-3) / 1e9
        return {"kernel": kernel, "us": round(t_ms * 1e3, 2), "achieved": round(a, 1), "unit": "GB/s",
                "frac": round(a / PEAK_HBM_GBPS, 4), "bytes_per_call": int(nbytes)}

    def mfma(t_ms, flop, kernel):
        a = flop / (t_ms * 1e-3) / 1e12
        return {"kernel": kernel, "us": round(t_ms * 1e3, 2), "achieved": round(a, 1), "unit": "TFLOP/s",
                "frac": round(a / PEAK_BF16_TFLOPS, 4), "flop_per_call": flop}

    out = {}
    sig = torch.full((1,), 0.6, dtype=torch.float32, device=dev)
    salt = torch.full((1,), 7, dtype=torch.int32, device=dev)
    g1 = gw.clone()
    t = _event_time_ms(lambda: pb.iso_noise_(g1, sigma=sig, salt_counter=salt), reps, torch)
    out["iso_noise"] = hbm(t, 6 * params, "noise_partials + noise_scale + noise_apply (6 B/param: the "
                           "gradient read twice and written once; the draws also pass through the workspace, 8 B/param more)")
    g2 = gw.clone()
    t = _event_time_ms(lambda: pb.sigmag_noise_(g2, dy, xb, sigma=sig, salt_counter=salt), reps, torch)
    out["sigmag_noise"] = mfma(t, 2.0 * M_TOK * N_OUT * K_IN,
                               "token_scale + token sum + WGRAD product (eps dy)^T x + sigmag partials / "
                               "scale / apply (bound by the extra 2 M N K product)")
    pk = layer.packed_w.clone()
    pb.set_prototype_semantics(True)
    pb.set_consolidate(dev, False)
    try:
        t = _event_time_ms(lambda: pb.apply_packed_adamw(
            pk, gw, None, layer.row_exp, layer.col_exp, layer._row_max_buf, layer._col_max_buf,
            lr=layer._lr_buf, eps=layer._eps_buf, gf_consol=50.0, v_scale=0.0, mass_preserve=True,
            v_row=layer.v_row, v_col=layer.v_col, sum_v_inv=layer._sum_v_inv, gf_trust_delta_sq=1.0,
            coh_pre=None, salt_prebumped=True), reps, torch)
    finally:
        pb.set_consolidate(dev, True)
        pb.set_prototype_semantics(False)
    out["proto_consf_update"] = hbm(t, UPDATE_BYTES_PER_PARAM * params,
                                    "apply_adamw_kernel (prototype semantics, accumulate step consf = 0)")
    cs = torch.empty(1, dtype=torch.float32, device=dev)
    ws = pb._stats_workspace(dev, CONFIG4_WATERMARKS, params)
    p = layer.packed_w
    # the stream is read at call time: the timer captures on its own stream
    t = _event_time_ms(lambda: C.check(C.lib().concord_coherence_sum(
        C.ptr(p), p.stride(0), N_OUT, K_IN, float(layer.drift_cancel_C), C.ptr(cs), C.ptr(ws), ws.numel(),
        C.stream_of(dev)), "coherence_sum"), reps, torch)
    out["coherence_meter"] = hbm(t, 4 * params, "coherence_partials + coherence_final (4 B/param)")
    nr = CONFIG4_WATERMARKS // 2
    nc = CONFIG4_WATERMARKS - nr
    wm = torch.randint(0, 30000, (CONFIG4_WATERMARKS,), dtype=torch.int32, device=dev)
    peak = torch.empty(1, dtype=torch.int32, device=dev)
    t = _event_time_ms(lambda: C.check(C.lib().concord_watermark_peak(
        C.ptr(wm), nr, C.ptr(wm[nr:]), nc, C.ptr(peak), C.ptr(ws), ws.numel(), C.stream_of(dev)),
        "watermark_peak"),
        reps, torch)
    out["watermark_peak"] = hbm(t, 4 * CONFIG4_WATERMARKS, "peak_partials + peak_final over config 4's "
                                f"{CONFIG4_WATERMARKS} row and column watermarks (4 B each)")
    # one training step of each SDXL 3 x 3 resnet conv shape at batch 2 of a
    # 1024 px latent (implicit-GEMM path: patches gathered inside the GEMMs
    # from channels-last activations): 6 M N K FLOP with M = B Ho Wo,
    # N = out channels, K = 9 in channels
    for cin, cout, hw in ((320, 320, 128), (640, 640, 64), (1280, 1280, 32)):
        conv = ca.ConcordConv2dPackedB(cin, cout, 3, padding=1, bias=True, device=dev, lr=5e-4)
        xc = torch.randn(2, cin, hw, hw, device=dev).to(torch.bfloat16).contiguous(
            memory_format=torch.channels_last).requires_grad_(True)
        dyc = (torch.randn(2, cout, hw, hw, device=dev) * 1e-3).to(torch.bfloat16).contiguous(
            memory_format=torch.channels_last)

        def cstep():
            xc.grad = None
            conv.bias.grad = None
            conv(xc).backward(dyc)
            conv.rebalance()

        for _ in range(3):
            cstep()
        torch.cuda.synchronize()
        t = _graph_ms(cstep, warmup, steps, torch)
        m = 2 * hw * hw
        key = "conv2d_3x3_step" if cin == 640 else f"conv2d_3x3_step_{cin}"
        out[key] = mfma(t, 6.0 * m * cout * cin * 9,
                        f"ConcordConv2dPackedB({cin}, {cout}, 3, padding 1) fwd + bwd + update + rebalance on "
                        f"(2, {cin}, {hw}, {hw}) channels-last, implicit GEMM; 6 M N K with M {m}, N {cout}, "
                        f"K {cin * 9}")
        del conv, xc, dyc
    return out


def _config4_groups(layers, xs, dys, reps, torch):
    """Per (out, in, tokens) group of config 4's layers: the layer step
    (forward, backward with the fused update) of every layer of the group
    captured in one HIP graph, replayed `reps` times; microseconds per layer
    and the group's share of 6 M N K."""
    groups = {}
    for la, m in layers:
        groups.setdefault((la.out_features, la.in_features, m), []).append(la)
    out = {}
    for (n_out, n_in, m), lays in groups.items():
        key = (m, n_in, n_out)
        x, dy = xs[key], dys[key]

        def run():
            for la in lays:
                x.grad = None
                la.bias.grad = None
                la(x).backward(dy)
        run()
        torch.cuda.synchronize()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                run()
        torch.cuda.current_stream().wait_stream(s)
        g.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps / len(lays)
        tf = 6.0 * m * n_out * n_in / (us * 1e-6) / 1e12
        # the layer step's binding roofline (no rebalance here: GatedRebalance
        # runs once per step): MFMA time of 6MNK or HBM time of its bytes
        hb = _step_hbm_bytes(n_out, n_in, m)
        t_roof = max(6.0 * m * n_out * n_in / (PEAK_BF16_TFLOPS * 1e12), hb / (PEAK_HBM_GBPS * 1e9))
        out[f"{n_in}to{n_out}_M{m}"] = {"layers": len(lays), "us_per_layer": round(us, 1),
                                         "group_ms": round(us * len(lays) / 1e3, 3), "tflops": round(tf, 1),
                                         "frac": round(tf / PEAK_BF16_TFLOPS, 4),
                                         "bound": ("hbm" if hb / (PEAK_HBM_GBPS * 1e9) >
                                                   6.0 * m * n_out * n_in / (PEAK_BF16_TFLOPS * 1e12) else "mfma"),
                                         "roofline_frac": round(t_roof / (us * 1e-6), 4)}
        del g
    return out


def _config4_step(steps, torch, ca, pb, per_group=False):
    """Config 4: one training step over all 754 SDXL Linear and 1x1 weights
    (2.25 B parameters held packed, 9.0 GB), each layer forward + backward
    (dgrad, wgrad, v-hat, fused update; winner flags) on its own token count,
    then GatedRebalance with the gate on the device.  The whole step is
    captured in one HIP graph and replayed; 6 M N K FLOP per layer."""
    from concord_amd.shapes import SDXL_1X1, SDXL_LINEAR
    dev = torch.device("cuda:0")
    torch.manual_seed(4)
    layers, flop, params = [], 0.0, 0
    for table in (SDXL_LINEAR, SDXL_1X1):
        for (n_out, n_in), count, m in table:
            for _ in range(count):
                lay = ca.ConcordLinearPackedB(n_in, n_out, bias=True, device=dev, lr=5e-4)
                lay.disable_cohpre()
                lay.gf_consol = 50.0
                layers.append((lay, m))
                flop += 6.0 * m * n_out * n_in
                params += n_out * n_in
    xs, dys = {}, {}
    for la, m in layers:
        key = (m, la.in_features, la.out_features)
        if key not in xs:
            xs[key] = torch.randn(m, la.in_features, device=dev).to(torch.bfloat16).requires_grad_(True)
            dys[key] = (torch.randn(m, la.out_features, device=dev) * 1e-3).to(torch.bfloat16)
    gate = ca.GatedRebalance([la for la, _ in layers])

    def step():
        for la, m in layers:
            key = (m, la.in_features, la.out_features)
            x = xs[key]
            x.grad = None
            la.bias.grad = None
            la(x).backward(dys[key])
        gate()

    step()   # creates the watermark buffers; the gate wires its slabs
    step()   # the gate builds its device plan
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    step()
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            step()
    torch.cuda.current_stream().wait_stream(s)
    g.replay()
    torch.cuda.synchronize()
    reps = max(2, min(steps, 5))
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    fires = gate.fires
    # the gate alone, no fire: watermarks zeroed, the device gate (two
    # launches of the peak, two of the group rebalance) against the host
    # gate (the peak, one host read, no rebalance launch)
    gate.row_all.zero_()
    gate.col_all.zero_()
    t_dev = _event_time_ms(gate, 20, torch)
    hg = ca.GatedRebalance([la for la, _ in layers], device_gate=False)
    hg.row_all, hg.col_all, hg._peak = gate.row_all, gate.col_all, gate._peak
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(20):
        hg()
    torch.cuda.synchronize()
    t_host = (time.perf_counter() - t0) * 1e3 / 20
    a = flop / (ms * 1e-3) / 1e12
    out = {"layers": len(layers), "params": params, "packed_GB": round(4 * params / 1e9, 2),
           "flop_per_step": flop, "ms_per_step": round(ms, 3), "tflops": round(a, 1),
           "frac": round(a / PEAK_BF16_TFLOPS, 4), "timing": f"one HIP graph per step, {reps} replays",
           "eager_ms_per_step": round(eager_ms, 1), "gate_fires_in_run": fires,
           "gate_nofire_us": {"device_gate": round(t_dev * 1e3, 1), "host_gate_with_item": round(t_host * 1e3, 1)}}
    if per_group:
        out["per_group"] = _config4_groups(layers, xs, dys, reps, torch)
    del g, layers, xs, dys, gate, hg
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def _step_hbm_bytes(N, K, M):
    """Algorithmic HBM bytes of one layer step: the packed words read by the
    forward and the dgrad (4 B each), the bf16 weight gradient written once
    and read by the update, the update's word read and write (10 B/param with
    the gradient read), and the activations: x read by the forward and the
    WGRAD, dx written; dy read by the dgrad and the WGRAD, y written."""
    return 20.0 * N * K + 6.0 * M * (N + K)


def _config3_steps(warmup, steps, torch, ca):
    """The same training step (fwd, dgrad, wgrad with v-hat, update with the
    winner flags, rebalance) on each config-3 shape; 6MNK FLOP per step.
    Each shape is priced against the roofline that bounds it: the MFMA time
    of its 6MNK FLOP or the HBM time of its algorithmic bytes
    (_step_hbm_bytes), whichever is longer (HBM for the few-token
    cross-attention shape)."""
    from concord_amd.shapes import CONFIG3
    out = {}
    dev = torch.device("cuda:0")
    for N, K, M in CONFIG3:
        torch.manual_seed(N + K + M)
        ly = ca.ConcordLinearPackedB(K, N, bias=True, device=dev, lr=5e-4)
        ly.disable_cohpre()
        ly.gf_consol = 50.0
        xs = torch.randn(M, K, device=dev).to(torch.bfloat16).requires_grad_(True)
        dys = (torch.randn(M, N, device=dev) * 1e-3).to(torch.bfloat16)

        def st():
            xs.grad = None
            ly.bias.grad = None
            ly(xs).backward(dys)
            ly.rebalance()

        for _ in range(3):
            st()
        torch.cuda.synchronize()
        t = _graph_ms(st, warmup, steps, torch)
        a = 6.0 * M * N * K / (t * 1e-3) / 1e12
        hb = _step_hbm_bytes(N, K, M)
        t_mfma = 6.0 * M * N * K / (PEAK_BF16_TFLOPS * 1e12)
        t_hbm = hb / (PEAK_HBM_GBPS * 1e9)
        out[f"{K}to{N}_M{M}"] = {"ms_per_step": round(t, 4), "tflops": round(a, 1),
                                 "frac": round(a / PEAK_BF16_TFLOPS, 4),
                                 "hbm_bytes": int(hb), "hbm_GBps": round(hb / (t * 1e-3) / 1e9, 1),
                                 "bound": "hbm" if t_hbm > t_mfma else "mfma",
                                 "roofline_frac": round(max(t_hbm, t_mfma) / (t * 1e-3), 4)}
    return out


def _weight_cache_step_ms(layer, x, dy, warmup, steps, torch, ca, per_graph=1):
    """The same step on a weight_cache=True copy of the layer, and on a fused
    copy made the same way, each timed twice in turn (fused, cache, fused,
    cache) so that both see the same state and clocks: (cache ms, fused ms),
    the means of the two timings each."""
    W = layer.get_weight().float()

    def timed(cache):
        wl = ca.ConcordLinearPackedB(K_IN, N_OUT, bias=True, device=x.device, lr=5e-4, weight_cache=cache)
        wl.disable_cohpre()
        wl.gf_consol = 50.0
        with torch.no_grad():
            wl.load_weights(W)

        def step():
            x.grad = None
            wl.bias.grad = None
            wl(x).backward(dy)
            wl.rebalance()

        for _ in range(3):
            step()
        return _graph_ms(step, warmup, steps, torch, per_graph)

    fused = [timed(False)]
    cache = [timed(True)]
    fused.append(timed(False))
    cache.append(timed(True))
    return sum(cache) / 2, sum(fused) / 2


def _dma_probe(reps, torch):
    """The load paths of the GEMM kernels, measured alone (concord_amd_diag.h):
    a 256 MiB copy through LDS-DMA loads (`reps` calls; its FETCH_SIZE /
    WRITE_SIZE per byte calibrate the counters of the LDS-DMA kernels), then
    the L2-to-CU rate: each workgroup streams its XCD's 1 MiB region 64 times
    (after the first pass every load hits that XCD's L2), by LDS-DMA and by
    register loads, 2 to 8 chunks of 16 KB in flight, one and two workgroups
    per CU.  Prints one JSON line; GB/s per CU = bytes / time / 256."""
    from concord_amd import _lib as C
    dev = torch.device("cuda:0")
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)

    def copy():   # on the current stream (the capture stream inside _event_time_ms)
        C.check(C.lib().concord_diag_dma_copy(C.ptr(a), C.ptr(b), a.numel(), C.stream_of(dev)), "diag_dma_copy")
    for _ in range(reps):
        copy()
    torch.cuda.synchronize()
    t_copy = _event_time_ms(copy, 5, torch)
    region, rep = 1 << 20, 64
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {"dma_copy_256MiB": {"us": round(t_copy * 1e3, 1), "GBps": round(2 * a.numel() / (t_copy * 1e-3) / 1e9, 1)},
           "l2_stream": {}}
    for lds_dma in (1, 0):
        for depth in (2, 4, 8):
            for per_cu in (1, 2):
                blocks = 256 * per_cu

                def run():
                    C.check(C.lib().concord_diag_l2_stream(C.ptr(a), region, rep, blocks, depth, lds_dma, C.ptr(sink),
                                                           C.stream_of(dev)), "diag_l2_stream")
                t = _event_time_ms(run, 3, torch)
                gbps_cu = blocks * region * rep / (t * 1e-3) / 1e9 / 256
                out["l2_stream"][f"{'dma' if lds_dma else 'vgpr'}_depth{depth}_wg{per_cu}"] = {
                    "us": round(t * 1e3, 1), "GBps_per_CU": round(gbps_cu, 1)}
    print(json.dumps({"dma_probe": out}), flush=True)


def _layer_ctx(layer, pb):
    """The attributes the backward's update reads from its autograd context,
    taken from the layer (the module's forward passes the same objects)."""
    import types
    return types.SimpleNamespace(
        packed_w=layer.packed_w, row_exp=layer.row_exp, col_exp=layer.col_exp, has_bias=True,
        optimizer_kind="adamw", weight_buf=None, lr=layer._lr_buf, mantissa_bias=layer.MANTISSA_BIAS,
        alpha=layer.alpha, beta1=layer.beta1, weight_decay=layer.weight_decay, eps=layer._eps_buf,
        step_cap=layer.step_cap, v_scale=layer.v_scale, precond_p=layer.precond_p, gf_consol=layer.gf_consol,
        drift_cancel_C=layer.drift_cancel_C, alpha_v_fast=layer.alpha_v_fast, wd_sv=layer.wd_sv, wd_sf=layer.wd_sf,
        mass_preserve=layer.mass_preserve_v, apply_chase=layer.apply_chase, track_rebalance=layer.track_rebalance,
        gf_trust_delta_sq=float(layer.gf_trust_delta_sq), coh_pre=layer._coh_pre, row_max_buf=layer._row_max_buf,
        col_max_buf=layer._col_max_buf, adafactor_beta2=float(layer.adafactor_beta2), v_row=layer.v_row,
        v_col=layer.v_col, sum_v_inv=layer._sum_v_inv)


def _bwd_update_fns(layer, xb, dy, pb):
    """The step's backward with its update, each way, as the module calls it
    (concord_dgrad_wgrad_update): (two_pass, fused).  two_pass = the separate
    launches (the default); fused = the finalize and the update in the WGRAD
    launch (set_fused_update)."""
    ctx = _layer_ctx(layer, pb)

    def two_pass():
        pb._dgrad_wgrad_update(ctx, dy, xb, False)

    def fused():
        pb._dgrad_wgrad_update(ctx, dy, xb, True)
    return two_pass, fused


def _fused_update_rows(layer, step, xb, dy, warmup, steps, G, reps, torch, pb):
    """The wgrad-fused update beside the two-pass form, measured in the same
    run on the same layer: the whole step (graph-timed as the headline, G
    steps per graph) and the backward entry with its update (events over a
    graph of `reps` calls), each way."""
    two_pass, fused = _bwd_update_fns(layer, xb, dy, pb)
    out = {}
    prev = pb._FUSED_UPDATE
    try:
        for name, on in (("two_pass", False), ("fused", True)):
            pb.set_fused_update(on)
            out[f"step_ms_{name}"] = round(_graph_ms(step, warmup, steps, torch, per_graph=G), 4)
        out["bwd_update_us_two_pass"] = round(_event_time_ms(two_pass, reps, torch) * 1e3, 2)
        out["bwd_update_us_fused"] = round(_event_time_ms(fused, reps, torch) * 1e3, 2)
        out["fused_launch_taken"] = bool(pb._LAST_FUSED[0])
        out["fault"] = pb.wgrad_update_faults(xb.device)
    finally:
        pb.set_fused_update(prev)
    out["kept"] = "fused" if prev else "two_pass"
    out["note"] = ("two_pass: gemm_dgt_kernel + gemm_tr_kernel<VH> (carrying the dgrad reduction) + "
                   "vhat_finalize_kernel (256-row totals) + apply_adamw_fast_kernel (1 / sum v_row from them); "
                   "fused: gemm_dgt_kernel + wgrad_update_kernel "
                   "(tiles, v-hat partials, grid barrier, finalize over the grid, grid barrier, update of each "
                   "tile from its accumulators; no bf16 weight gradient)")
    return out


def _only(which, reps, layer, xb, dy, torch, pb):
    """Run one kernel of the step `reps` times (profiling entry)."""
    st = (layer.packed_w, layer.row_exp, layer.col_exp)
    dev = xb.device
    if which == "copy":
        a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        fn = lambda: b.copy_(a)  # noqa: E731
    elif which == "dma":
        _dma_probe(reps, torch)
        return
    elif which in ("bwd_update", "bwd_update_fused"):
        two_pass, fused = _bwd_update_fns(layer, xb, dy, pb)
        fn = fused if which == "bwd_update_fused" else two_pass
    elif which == "fwd":
        fn = lambda: pb._gemm_fwd(xb, *st, 15, layer.bias, None)  # noqa: E731
    elif which == "dgrad":
        fn = lambda: pb._gemm_dgrad(dy, *st, 15, None)  # noqa: E731
    elif which == "wgrad":
        fn = lambda: pb._wgrad(dy, xb)  # noqa: E731
    elif which == "bwd":
        fn = lambda: pb._dgrad_wgrad_vhat(dy, xb, *st, 15, layer.v_row, layer.v_col,  # noqa: E731
                                          layer._sum_v_inv, 0.999, layer._row_max_buf, layer._col_max_buf,
                                          None, with_bias=True)
    elif which == "ns5":
        g5 = (torch.randn(N_OUT, K_IN, device=dev) * 1e-3).to(torch.bfloat16)
        o5 = torch.empty_like(g5)
        fn = lambda: pb.muon_ns5(g5, out=o5)  # noqa: E731
    elif which == "wgrad_vhat":
        fn = lambda: pb._wgrad_vhat(dy, xb, layer.v_row, layer.v_col, layer._sum_v_inv, 0.999,  # noqa: E731
                                    layer._row_max_buf, layer._col_max_buf, None, with_bias=True)
    else:
        gw = pb._wgrad(dy, xb)
        if which == "vhat":
            fn = lambda: pb.vhat_ema(gw, layer.v_row, layer.v_col, layer._sum_v_inv)  # noqa: E731
        elif which == "update":
            pk = layer.packed_w.clone()
            fn = lambda: pb.apply_packed_adamw(  # noqa: E731
                pk, gw, None, layer.row_exp, layer.col_exp, layer._row_max_buf, layer._col_max_buf,
                lr=layer._lr_buf, eps=layer._eps_buf, gf_consol=50.0, v_scale=0.0, mass_preserve=True,
                v_row=layer.v_row, v_col=layer.v_col, sum_v_inv=layer._sum_v_inv, gf_trust_delta_sq=1.0,
                coh_pre=None, salt_prebumped=True)
        else:
            wbuf = torch.empty((N_OUT, K_IN), dtype=torch.bfloat16, device=dev)
            fn = lambda: pb.materialize_packed_bf16(*st, wbuf)  # noqa: E731
    for _ in range(reps):
        fn()
    torch.cuda.synchronize()
    print(json.dumps({"only": which, "reps": reps}))


def _child_pids():
    """Process ids whose parent is this process (from /proc)."""
    pids = []
    try:
        for tid in os.listdir("/proc/self/task"):
            with open(f"/proc/self/task/{tid}/children") as f:
                pids += [int(p) for p in f.read().split()]
    except OSError:
        pass
    return sorted(set(pids))


def _reap_children(limit_s=5.0):
    """Name on stderr any child process still running at the end and wait
    up to limit_s for it, so the script does not leave one behind."""
    pids = _child_pids()
    for pid in pids:
        try:
            with open(f"/proc/{pid}/cmdline", "rb") as f:
                cmd = f.read().replace(b"\0", b" ").decode(errors="replace").strip()
        except OSError:
            cmd = "?"
        print(f"bench: child process {pid} still running at exit: {cmd}", file=sys.stderr)
    t0 = time.monotonic()
    while pids and time.monotonic() - t0 < limit_s:
        left = []
        for pid in pids:
            try:
                done, _ = os.waitpid(pid, os.WNOHANG)
            except ChildProcessError:
                continue
            if done == 0:
                left.append(pid)
        pids = left
        if pids:
            time.sleep(0.1)


def _make_step(torch, ca, dev):
    """The headline layer (seed 0) and its training step."""
    torch.manual_seed(0)
    layer = ca.ConcordLinearPackedB(K_IN, N_OUT, bias=True, device=dev, lr=5e-4)
    ca.set_ratio_coh(True)
    ca.set_ratio_coh_floors(0.9, 0.999)
    layer.disable_cohpre()
    layer.gf_consol = 50.0
    x = torch.randn(M_TOK, K_IN, device=dev).to(torch.bfloat16).requires_grad_(True)
    dy = (torch.randn(M_TOK, N_OUT, device=dev) * 1e-3).to(torch.bfloat16)

    def step():
        # gradients of the input and the bias go to the caller (set to None as
        # optimizer.zero_grad(set_to_none=True) does; no accumulate kernel)
        x.grad = None
        layer.bias.grad = None
        y = layer(x)
        y.backward(dy)
        layer.rebalance()

    for _ in range(3):
        step()
    torch.cuda.synchronize()
    return layer, x, dy, step


def _capture_steps(step, G, torch):
    """(run, steps per run, mode): G >= 1 steps captured in one HIP graph, or
    the eager step when G is 0 or the capture fails."""
    if G < 1:
        return step, 1, "eager"
    try:
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                step()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for _ in range(G):
                step()
        torch.cuda.synchronize()
        return g.replay, G, (f"hipgraph ({G} steps per graph)" if G > 1 else "hipgraph")
    except Exception as exc:  # capture unsupported: time eagerly
        print(f"bench.py: graph capture failed ({exc}); timing eager steps", file=sys.stderr)
        torch.cuda.synchronize()
        return step, 1, "eager"


def _timed_steps(run, warm_runs, timed_runs, torch):
    """(ms, wall s) of `timed_runs` calls of run after `warm_runs` untimed ones,
    HIP events on the launching stream, synchronized on both sides."""
    for _ in range(warm_runs):
        run()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(timed_runs):
        run()
    ev1.record()
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1), time.perf_counter() - t0


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # the untimed warmup runs the layer into its steady state: the first steps
    # after init tick many exponents at once, and the clocks settle
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-next-rows", action="store_true",
                    help="skip the context timings of the rows beside the step (keeps a kernel profile to the "
                         "step's own shapes)")
    ap.add_argument("--no-config4", action="store_true",
                    help="skip the config-4 row (the graph-captured step over all 754 SDXL weights)")
    ap.add_argument("--only", default=None,
                    choices=["fwd", "bwd", "dgrad", "wgrad", "wgrad_vhat", "vhat", "update", "materialize",
                             "copy", "dma", "ns5", "config3", "config4", "bwd_update", "bwd_update_fused"],
                    help="time one entry alone; config3 times only the step on each config-3 SDXL shape; "
                         "config4 only the config-4 step, and each of its (shape, tokens) groups of layers")
    ap.add_argument("--reps", type=int, default=20)
    ap.add_argument("--graph-steps", type=int, default=5,
                    help="training steps captured per HIP graph (1 = one graph replay per step)")
    ap.add_argument("--clock-warmup", type=float, default=0.5,
                    help="seconds of training steps on a scratch layer (same shape, same init) run right "
                         "before the timed layer's warmup, so the timed steps run at settled clocks "
                         "(0 = none)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the packed path runs on one GPU; it has no multi-GPU mode)", file=sys.stderr)
        sys.exit(2)

    import torch
    import concord_amd as ca
    from concord_amd import packed_b as pb

    dev = torch.device("cuda:0")
    layer, x, dy, step = _make_step(torch, ca, dev)

    if args.only == "config3":
        print(json.dumps({"sdxl_shapes": _config3_steps(args.warmup, args.steps, torch, ca)}), flush=True)
        return
    if args.only == "config4":
        del layer, x, dy
        torch.cuda.empty_cache()
        print(json.dumps({"config4_step": _config4_step(args.steps, torch, ca, pb, per_group=True)}), flush=True)
        return
    if args.only:
        _only(args.only, args.reps, layer, x.detach(), dy, torch, pb)
        return

    # G consecutive steps per graph (G divides the step counts), so the replay
    # launch overhead is paid once per G steps, as a training loop that
    # captures its inner steps does; every step's kernels all run
    G = 1
    if not args.no_graph:
        G = max(1, args.graph_steps)
        while G > 1 and (args.steps % G or args.warmup % G):
            G -= 1
    run, per_run, mode = _capture_steps(step, G, torch)

    # The clocks: after the process start and the layer's set-up the device has
    # been mostly idle, and its clocks rise over the next ~40 ms of steady work
    # (measured: a 5-step graph replay 176-180 us per step at first, 155 us
    # after ~40 replays, back to 176 us after a 2 s pause, 156 us at once when a
    # 0.5 s busy spell precedes it).  A scratch layer of the same shape and
    # init, timed first exactly as the headline is (W warmup, K timed steps),
    # gives the figure before the clocks settle; then its steps run for
    # --clock-warmup seconds, and the headline layer's W warmup and K timed
    # steps follow at once.  The headline layer itself runs exactly W steps
    # before its timed K.
    ms_cold = None
    if args.clock_warmup > 0:
        s_layer, _, _, s_step = _make_step(torch, ca, dev)
        s_run, _, _ = _capture_steps(s_step, per_run, torch)
        ms_cold = _timed_steps(s_run, args.warmup // per_run, args.steps // per_run, torch)[0] / args.steps
        t_end = time.perf_counter() + args.clock_warmup
        while time.perf_counter() < t_end:
            for _ in range(8):
                s_run()
            torch.cuda.synchronize()
        for _ in range(8):
            s_run()   # still running when the headline layer's warmup is queued
    ms_total, wall = _timed_steps(run, args.warmup // per_run, args.steps // per_run, torch)
    ms_step = ms_total / args.steps
    if args.clock_warmup > 0:
        del s_layer, s_step, s_run
    flops_step = 6.0 * M_TOK * N_OUT * K_IN
    value = flops_step / (ms_step * 1e-3) / 1e12

    # per-entry averages (HIP events on the stream the kernels run on), each the
    # call the step makes: forward, dgrad, wgrad + v-hat + bias gradient, update
    xb = x.detach()
    st = (layer.packed_w, layer.row_exp, layer.col_exp)
    reps = 20
    t_fwd = _event_time_ms(lambda: pb._gemm_fwd(xb, *st, 15, layer.bias, None), reps, torch)
    t_dgrad = _event_time_ms(lambda: pb._gemm_dgrad(dy, *st, 15, None), reps, torch)
    t_wgv = _event_time_ms(lambda: pb._wgrad_vhat(dy, xb, layer.v_row, layer.v_col, layer._sum_v_inv, 0.999,
                                                  layer._row_max_buf, layer._col_max_buf, None,
                                                  with_bias=True), reps, torch)
    t_wgrad = _event_time_ms(lambda: pb._wgrad(dy, xb), reps, torch)
    t_bwd = _event_time_ms(lambda: pb._dgrad_wgrad_vhat(dy, xb, *st, 15, layer.v_row, layer.v_col,
                                                        layer._sum_v_inv, 0.999, layer._row_max_buf,
                                                        layer._col_max_buf, None, with_bias=True),
                           reps, torch)
    gw = pb._wgrad(dy, xb)
    pk_copy = layer.packed_w.clone()
    t_vhat = _event_time_ms(lambda: pb.vhat_ema(gw, layer.v_row, layer.v_col, layer._sum_v_inv),
                            reps, torch)

    def upd():
        pb.apply_packed_adamw(pk_copy, gw, None, layer.row_exp, layer.col_exp, layer._row_max_buf,
                              layer._col_max_buf, lr=layer._lr_buf, eps=layer._eps_buf, gf_consol=50.0,
                              v_scale=0.0, mass_preserve=True, v_row=layer.v_row, v_col=layer.v_col,
                              sum_v_inv=layer._sum_v_inv, gf_trust_delta_sq=1.0, coh_pre=None,
                              salt_prebumped=True)
    t_upd = _event_time_ms(upd, reps, torch)
    fused_rows = _fused_update_rows(layer, step, xb, dy, args.warmup, args.steps, per_run, reps, torch, pb)
    wbuf = torch.empty((N_OUT, K_IN), dtype=torch.bfloat16, device=dev)
    t_mat = _event_time_ms(lambda: pb.materialize_packed_bf16(layer.packed_w, layer.row_exp,
                                                              layer.col_exp, wbuf), reps, torch)
    # config 5's Muon drive on this layer's gradient (context: NS5 = 5 x
    # (2 m^2 n + 2 m^3 + 2 m^2 n) FLOP with m = 1280, n = 5120)
    ns5_out = torch.empty_like(gw)
    t_ns5 = _event_time_ms(lambda: pb.muon_ns5(gw, out=ns5_out), reps, torch)
    ns5_flop = 5.0 * (4.0 * K_IN * K_IN * N_OUT + 2.0 * K_IN ** 3)
    # no-fire rebalance: zeroed watermarks, so no row or column ticks
    layer._row_max_buf.zero_()
    layer._col_max_buf.zero_()
    t_reb = _event_time_ms(layer.rebalance, reps, torch)
    next_rows = {} if args.no_next_rows else _next_rows(layer, xb, dy, gw, reps, args.warmup, args.steps, torch,
                                                           ca, pb)
    sdxl_shapes = {} if args.no_next_rows else _config3_steps(args.warmup, args.steps, torch, ca)
    config4 = None if args.no_config4 else _config4_step(args.steps, torch, ca, pb)

    # the reference's own dataflow on the same workload, for context: the
    # update emits the bf16 weight (materialize-merge) and the next step's
    # forward and dgrad are bf16 GEMMs on it (this library's kernels)
    Wd0 = layer.get_weight()
    t_bf_fwd = _event_time_ms(lambda: pb._gemm_fwd(xb, None, None, None, 15, layer.bias, Wd0), reps, torch)
    t_bf_dgrad = _event_time_ms(lambda: pb._gemm_dgrad(dy, None, None, None, 15, Wd0), reps, torch)
    wc_ms, wc_fused_ms = _weight_cache_step_ms(layer, x, dy, args.warmup, args.steps, torch, ca, per_run)

    # library reference (hipBLASLt through torch.matmul) on the same bf16 shapes,
    # for context only: W decoded once, not part of the measured path
    Wd = layer.get_weight()
    t_lib_fwd = _event_time_ms(lambda: torch.matmul(xb, Wd.t()), reps, torch)
    t_lib_dgrad = _event_time_ms(lambda: torch.matmul(dy, Wd), reps, torch)
    t_lib_wgrad = _event_time_ms(lambda: torch.matmul(dy.t(), xb), reps, torch)

    gemm_flop = 2.0 * M_TOK * N_OUT * K_IN
    fwd_tflops = gemm_flop / (t_fwd * 1e-3) / 1e12
    params = N_OUT * K_IN
    upd_gbps = UPDATE_BYTES_PER_PARAM * params / (t_upd * 1e-3) / 1e9
    traffic = _read_traffic()

    def gemm_roof(key, name, t_ms):
        a = gemm_flop / (t_ms * 1e-3) / 1e12
        return {"bound": "mfma", "kernel": name, "achieved": round(a, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(a / PEAK_BF16_TFLOPS, 4), "traffic": traffic.get(key),
                "us": round(t_ms * 1e3, 2)}

    def hbm_roof(key, name, t_ms, nbytes):
        a = nbytes / (t_ms * 1e-3) / 1e9
        return {"bound": "hbm", "kernel": name, "achieved": round(a, 1), "peak": PEAK_HBM_GBPS,
                "unit": "GB/s", "frac": round(a / PEAK_HBM_GBPS, 4), "traffic": traffic.get(key),
                "us": round(t_ms * 1e3, 2)}

    def bwd_roof(key, name, t_ms):
        r = gemm_roof(key, name, t_ms)
        a = 2.0 * gemm_flop / (t_ms * 1e-3) / 1e12
        r.update(achieved=round(a, 2), frac=round(a / PEAK_BF16_TFLOPS, 4))
        return r

    roofs = {
        "dqgemm_fwd": gemm_roof("dqgemm_fwd", "gemm_dma_kernel<FWD, 256, 160> (fused dequant-GEMM forward)",
                                t_fwd),
        "bwd_products": bwd_roof("bwd_products", "gemm_dgt_kernel<DGRAD, 256, 128> + gemm_tr_kernel<256, 128, "
                                 "4, 2, VH> carrying the dgrad's split-K reduction + vhat_finalize_kernel "
                                 "(concord_dgrad_wgrad_vhat, the step's two products and v-hat EMA, which the step runs through "
                                 "concord_dgrad_wgrad_update before its update; 4 M N K FLOP)", t_bwd),
        "dqgemm_dgrad": gemm_roof("dqgemm_dgrad", "gemm_dgt_kernel<DGRAD, 256, 128> + splitk_reduce_kernel "
                                  "(fused dequant-GEMM dgrad, 3-way split reduction)", t_dgrad),
        "wgrad_vhat": gemm_roof("wgrad_vhat", "gemm_tr_kernel<256, 128, 4, 2, VH> + vhat_finalize_kernel "
                                "(wgrad with v-hat partials and bias gradient in the epilogue, then the "
                                "v-hat EMA and its row sum)", t_wgv),
        "apply_adamw": hbm_roof("apply_adamw", "apply_adamw_fast_kernel<ratio> (packed update, winner flags)",
                                t_upd, UPDATE_BYTES_PER_PARAM * params),
    }
    # the update is bound by VALU issue, not HBM: its fraction of the VALU
    # peak from the committed lane-instructions per word (SQ_INSTS_VALU), with
    # the HBM figures kept beside it
    vpw = _read_valu_per_word()
    upd_hbm = dict(roofs["apply_adamw"])
    if vpw:
        a_valu = params * vpw / (t_upd * 1e-3) / 1e12
        roofs["apply_adamw"] = {
            "bound": "valu", "kernel": upd_hbm["kernel"], "achieved": round(a_valu, 2),
            "peak": round(PEAK_VALU_TLANE_OPS, 2), "unit": "Tlane-op/s",
            "frac": round(a_valu / PEAK_VALU_TLANE_OPS, 4), "valu_lane_instr_per_word": vpw,
            "hbm_achieved_GBps": upd_hbm["achieved"], "hbm_frac": upd_hbm["frac"],
            "traffic": upd_hbm["traffic"], "us": upd_hbm["us"]}
    # the longest entry the step calls (dgrad and wgrad_vhat alone are context:
    # the step runs them as bwd_products)
    step_entries = ("dqgemm_fwd", "bwd_products", "apply_adamw")
    dominant = max(step_entries, key=lambda k: roofs[k]["us"])

    out = {
        "metric": "dequant-matmul TFLOP/s (%MFMA peak) + packed-update GB/s (%HBM), SDXL linears",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "sdxl_linear_1280to5120_M2048_fwd_dgrad_wgrad_update_rebalance",
                   "N": N_OUT, "K": K_IN, "M": M_TOK, "optimizer": "winner (ratio_coh, gf_consol=50)",
                   "forward": "fused dequant-GEMM", "timing": mode},
        "clock_warmup": {"s": args.clock_warmup,
                         "ms_per_step_before": None if ms_cold is None else round(ms_cold, 4),
                         "note": "ms_per_step_before: a scratch layer of the same shape and init timed exactly "
                                 "as the headline (W warmup, K timed steps) before the clock warm-up; the "
                                 "headline layer runs W steps, then its K timed steps, right after the scratch "
                                 "layer's steps have run for s seconds"},
        "roofline": dict(upd_hbm if dominant == "apply_adamw" else roofs[dominant], step_kernel=dominant),
        "rooflines": roofs,
        "kernel_us": {"dqgemm_fwd": round(t_fwd * 1e3, 2), "bwd_products": round(t_bwd * 1e3, 2),
                      "dqgemm_dgrad": round(t_dgrad * 1e3, 2),
                      "wgrad_vhat": round(t_wgv * 1e3, 2), "wgrad_alone": round(t_wgrad * 1e3, 2),
                      "vhat_ema_alone": round(t_vhat * 1e3, 2),
                      "apply_adamw": round(t_upd * 1e3, 2), "materialize": round(t_mat * 1e3, 2),
                      "rebalance_nofire": round(t_reb * 1e3, 2)},
        "gemm_tflops": {"fwd": round(fwd_tflops, 1),
                        "bwd_products": round(2.0 * gemm_flop / (t_bwd * 1e-3) / 1e12, 1),
                        "dgrad": round(gemm_flop / (t_dgrad * 1e-3) / 1e12, 1),
                        "wgrad_vhat": round(gemm_flop / (t_wgv * 1e-3) / 1e12, 1),
                        "wgrad_alone": round(gemm_flop / (t_wgrad * 1e-3) / 1e12, 1)},
        "materialize_GBps": round(DECODE_BYTES_PER_PARAM * params / (t_mat * 1e-3) / 1e9, 1),
        "wgrad_fused_update": fused_rows,
        "muon_ns5": {"us": round(t_ns5 * 1e3, 1),
                     "tflops": round(ns5_flop / (t_ns5 * 1e-3) / 1e12, 1)},
        "next_rows": dict(note="the rows beside the step, timed on the same state; context only",
                          **next_rows),
        "sdxl_shapes": dict(note="the same step on each config-3 SDXL linear shape (out N, in K, tokens M); "
                                 "context only", **sdxl_shapes),
        "config4_step": dict(note="config 4: one training step over the 754 SDXL Linear + 1x1 weights with "
                                  "GatedRebalance (device gate), one HIP graph; context only",
                             **(config4 or {})),
        "weight_cache_mode": {
            "note": "the reference's dataflow (update emits the bf16 weight; forward and dgrad are bf16 "
                    "GEMMs on it), same workload; context only. fused_ms_per_step: the fused step on a "
                    "copy made and timed the same way, alternating with the cache copy (same state and "
                    "clocks; the headline above is timed first, right after the layer's init)",
            "ms_per_step": round(wc_ms, 4),
            "tflops": round(flops_step / (wc_ms * 1e-3) / 1e12, 2),
            "fused_ms_per_step": round(wc_fused_ms, 4),
            "fused_tflops": round(flops_step / (wc_fused_ms * 1e-3) / 1e12, 2),
            "fwd_us": round(t_bf_fwd * 1e3, 2), "dgrad_us": round(t_bf_dgrad * 1e3, 2)},
        "library_bf16_gemm_tflops": {
            "note": "torch.matmul (hipBLASLt) on a pre-decoded bf16 W, same shapes; context only",
            "fwd": round(gemm_flop / (t_lib_fwd * 1e-3) / 1e12, 1),
            "dgrad": round(gemm_flop / (t_lib_dgrad * 1e-3) / 1e12, 1),
            "wgrad": round(gemm_flop / (t_lib_wgrad * 1e-3) / 1e12, 1)},
        "wall_s_timed": round(wall, 3),
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    _reap_children()


if __name__ == "__main__":
    main()
