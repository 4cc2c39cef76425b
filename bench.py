"""Benchmark of the MoE block on one MI355X (BASELINE.json's metric on its configs).

A step is one forward of the block (router, experts, shared expert, combine) over one batch of synthetic tokens,
inputs resident in HBM. The default run measures both halves of BASELINE's metric and prints them in one JSON line:
  - decode (the line's value): BASELINE.json configs[1] (config 2), the speculative-verify batch of 8 tokens, Q4_K
    experts, hidden 2048, 512 experts, top-10 + shared, intermediate 512, Zipf(1.1) logit bias; roofline: HBM GB/s;
  - prefill (the "prefill" object): config 4, one 2048-token chunk, Q4_K, Zipf(1.1); roofline: the routed gate/up
    launch's int8 MFMA rate.
Each has a cpu_baseline: oracle/cpu_fast.c (the oracle's bits, SIMD integer dots, OpenMP) timed on this host's
physical cores and on one core, the median of 20 or more repetitions.

Cache defeat (decode): the MI355X's 256 MB Infinity Cache would hold one layer's touched weights, so the block is
resident as several layers (independent routers and biases, so each step routes differently) whose touched bytes,
counted from each layer's own routing, sum past 512 MB; step i runs layer i mod n_layers.

--config picks one of BASELINE's configs alone: decode 1, 2, 3, 3b; prefill 4; the 48-layer stack 5 (decode) and
5p (prefill, two chunks of 2048).
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

CONFIGS = {
    "1": dict(name="config1: decode T=1, Q8_0", types=(8, 8, 8, 8), T=1, zipf=None),
    "2": dict(name="config2: verify T=8, Q4_K, Zipf(1.1)", types=(12, 12, 12, 12), T=8, zipf=1.1),
    "3": dict(name="config3: decode T=1, IQ3_S", types=(21, 21, 21, 21), T=1, zipf=None),
    "3b": dict(name="config3: decode T=4, IQ3_S", types=(21, 21, 21, 21), T=4, zipf=None),
    "4": dict(name="config4: prefill T=2048, Q4_K, Zipf(1.1)", types=(12, 12, 12, 12), T=2048, zipf=1.1),
    "5": dict(name="config5: 48-layer stack, decode T=1, gate/up IQ3_S, down Q4_K, shared Q8_0, Zipf(1.1) per layer",
              types=(21, 12, 8, 8), T=1, zipf=1.1, layers=48),
    "5p": dict(name="config5: 48-layer stack, prefill 4096 tokens in 2 chunks of 2048, gate/up IQ3_S, down Q4_K, "
                    "shared Q8_0, Zipf(1.1) per layer", types=(21, 12, 8, 8), T=4096, chunk=2048, zipf=1.1, layers=48),
    # Not a BASELINE config: config 4's block with the hyper-connection mix and combine around it (moe_forward_hc), a
    # low rank of 256 at this n_embd (the model's 320 at 2560 scaled); its own JSON line, never the headline.
    "hc": dict(name="config4 + hyper-connection mix and combine (hc_lr 256): prefill T=2048, Q4_K, Zipf(1.1)",
               types=(12, 12, 12, 12), T=2048, zipf=1.1, hc_lr=256),
    "hc2": dict(name="config2 + hyper-connection mix and combine (hc_lr 256): verify T=8, Q4_K, Zipf(1.1)",
                types=(12, 12, 12, 12), T=8, zipf=1.1, hc_lr=256),
}
FP64_PEAK_TFLOPS = 78.6  # dense fp64 MFMA, MI355X
H, F, E, K = 2048, 512, 512, 10
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, MI355X
# The routed gate/up kernel of a gate type (the launch the prefill roofline is quoted on); pf_gemm16 for the others.
GU_KERNEL = {12: "pf_gate_up_q4k", 21: "pf_gate_up_iq3s"}  # Q4_K, IQ3_S


class Hip:
    """The few HIP runtime calls the bench needs for its own device buffers."""

    def __init__(self):
        self.rt = C.CDLL("libamdhip64.so")
        self.rt.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.rt.hipFree.argtypes = [C.c_void_p]
        self.rt.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.rt.hipDeviceSynchronize.argtypes = []

    def malloc(self, n):
        p = C.c_void_p()
        assert self.rt.hipMalloc(C.byref(p), n) == 0, "hipMalloc"
        return p

    def h2d(self, dst, a):
        assert self.rt.hipMemcpy(dst, a.ctypes.data_as(C.c_void_p), a.nbytes, 1) == 0

    def d2h(self, a, src):
        assert self.rt.hipMemcpy(a.ctypes.data_as(C.c_void_p), src, a.nbytes, 2) == 0

    def sync(self):
        assert self.rt.hipDeviceSynchronize() == 0

    def event(self):
        e = C.c_void_p()
        assert self.rt.hipEventCreate(C.byref(e)) == 0, "hipEventCreate"
        return e

    def record(self, e, stream):
        assert self.rt.hipEventRecord(e, C.c_void_p(stream)) == 0, "hipEventRecord"

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        assert self.rt.hipEventElapsedTime(C.byref(ms), a, b) == 0, "hipEventElapsedTime"
        return ms.value


def timed_steps(hip, blk, steps_once, launches):
    """The timed region of a decode run: the K steps bracketed by synchronisations, with one HIP event before and one
    after them on the stream the kernel is launched on (the block's). moe_decode is the only kernel in the region, so
    the events' elapsed time over its `launches` launches is its average launch duration (the gaps between launches
    included). Events around every launch would put their own packets between the launches and slow the job."""
    stream = blk.stream()
    ea, eb = hip.event(), hip.event()
    hip.sync()
    t0 = time.perf_counter()
    hip.record(ea, stream)
    steps_once()
    hip.record(eb, stream)
    hip.sync()
    t1 = time.perf_counter()
    return t0, t1, {"moe_decode": hip.elapsed_ms(ea, eb) / launches}, launches


def timed_steps_per_launch(hip, blk, steps_once):
    """The timed region of a prefill run: the K steps bracketed by synchronisations, with HIP events on the block's
    stream around each gate/up launch only (the roofline's kernel; every event pair adds packets between launches).
    The same K steps then run again, untimed, with events around every kernel for the per-kernel breakdown; the
    gate/up average reported is the timed region's."""
    blk.set_timing(2)
    hip.sync()
    t0 = time.perf_counter()
    steps_once()
    hip.sync()
    t1 = time.perf_counter()
    kt_timed, nf = blk.kernel_times()
    blk.set_timing(True)
    steps_once()
    hip.sync()
    ktimes, _ = blk.kernel_times()
    blk.set_timing(False)
    ktimes.update(kt_timed)
    return t0, t1, ktimes, nf


def measured_traffic(config):
    """HBM bytes per moe_decode launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes (copy-calibrated) and
    recorded in profiles/traffic_moe_decode.json with the commands that made them; None if not measured."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic_moe_decode.json")) as f:
            return json.load(f)["moe_decode"][config]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def measured_prefill_traffic(config):
    """HBM bytes per routed gate/up launch (copy-calibrated FETCH_SIZE + WRITE_SIZE) recorded in
    profiles/traffic_prefill.json; None if not measured for this config."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic_prefill.json")) as f:
            return json.load(f)["pf_gate_up"][config]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_host():
    """The host the CPU baseline runs on: its model, its physical cores among the CPUs this process may use, and the
    thread count used (one a physical core)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    allowed = sorted(os.sched_getaffinity(0))
    cores = set()
    try:
        import subprocess
        out = subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET"], stdout=subprocess.PIPE, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("#"):
                continue
            cpu, core, sock = (int(v) for v in line.split(",")[:3])
            if cpu in allowed:
                cores.add((sock, core))
    except Exception:
        pass
    physical = len(cores) if cores else len(allowed)
    return {"model": model, "physical_cores": physical, "allowed_cpus": len(allowed)}


def cpu_median(fn, reps=20, max_s=20.0):
    """Median seconds of fn over at least `reps` calls (stopping early, with at least 3, past max_s)."""
    ts = []
    t_all = time.perf_counter()
    while len(ts) < reps:
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
        if time.perf_counter() - t_all > max_s and len(ts) >= 3:
            break
    ts.sort()
    return ts[len(ts) // 2], len(ts)


def cpu_baseline(h, layer, x, unit_per_token, unit, check=None, one_core_tokens=None):
    """oracle/cpu_fast.c on this host: all physical cores and one core, medians of >= 20 repetitions on the sample x
    (the first one_core_tokens rows for the one-core figure). unit_per_token converts tokens/s into the metric's
    second unit (GB/s or TFLOP/s). check: y the GPU gave for x, compared bit for bit."""
    info = cpu_host()
    n = max(1, info["physical_cores"])
    y, _, _ = h.fast_forward(layer, x, nthreads=n)  # warm: the router transpose, page-in
    same = None if check is None else bool(np.array_equal(y, check))
    med, reps = cpu_median(lambda: h.fast_forward(layer, x, nthreads=n))
    x1 = x if one_core_tokens is None else x[:one_core_tokens]
    med1, reps1 = cpu_median(lambda: h.fast_forward(layer, x1, nthreads=1), max_s=15.0)
    T, T1 = x.shape[0], x1.shape[0]
    return {"value": round(T / med, 2), "unit": "tokens/s", "cores": n, "kind": "port",
            "isa": h.oracle.orc_fast_isa().decode(), "cpu_model": info["model"],
            "allowed_cpus": info["allowed_cpus"],
            "second_unit": {unit: round(unit_per_token * T / med, 3)},
            "one_core": {"value": round(T1 / med1, 2), "unit": "tokens/s", unit: round(unit_per_token * T1 / med1, 3),
                         "reps": reps1, "tokens": T1},
            "reps": reps, "equals_gpu_y": same,
            "sample": "%d tokens a forward, median of %d forwards on %d threads (one a physical core) by "
                      "oracle/cpu_fast.c: the oracle's arithmetic, bit for bit, with %s integer dot products"
                      % (T, reps, n, h.oracle.orc_fast_isa().decode())}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="default 2000 (decode), 100 (prefill)")
    ap.add_argument("--warmup", type=int, default=None, help="default 200 (decode), 10 (prefill)")
    ap.add_argument("--config", default=None, choices=sorted(CONFIGS),
                    help="one config alone; default: config 2 (decode, the line's value) and config 4 (prefill)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="the 48-layer stack's CPU sample length")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run five 256 MiB device-to-device copies (the reference transfer for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE passes) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        hip = Hip()
        n = 256 << 20
        a, b = hip.malloc(n), hip.malloc(n)
        for _ in range(5):
            assert hip.rt.hipMemcpy(b, a, n, 3) == 0
        hip.sync()
        return
    if args.gpus != 1:
        print("bench.py: this build measures one GPU only (the MoE block on one MI355X); --gpus %d is not run"
              % args.gpus, file=sys.stderr)
        sys.exit(2)

    import c0ven_amd as moe
    from tests import harness as h

    if args.config is None:
        out = decode(args, CONFIGS["2"], "2", moe, h)
        pf = prefill(args, CONFIGS["4"], "4", moe, h)
        out["prefill"] = {k: pf[k] for k in ("value", "unit", "ms_per_step", "steps", "warmup", "config", "roofline",
                                             "block", "parity", "cpu_baseline")}
        out["prefill"]["metric"] = "MoE block tokens/s and TFLOP/s (prefill, config 4)"
        print(json.dumps(out), flush=True)
        return
    cfg = CONFIGS[args.config]
    if "layers" in cfg:
        return stack(args, cfg, moe, h)
    if "hc_lr" in cfg:
        return hc(args, cfg, moe, h)
    out = (prefill if cfg["T"] > 16 else decode)(args, cfg, args.config, moe, h)
    print(json.dumps(out), flush=True)


def decode(args, cfg, key, moe, h):
    """A decode config (T <= 16): one launch of moe_decode a step, layers resident past 512 MB of touched weights."""
    gt, dt, sgt, sdt = cfg["types"]
    T = cfg["T"]
    steps = 2000 if args.steps is None else args.steps
    warmup = 200 if args.warmup is None else args.warmup
    hip = Hip()
    t_setup = time.time()
    # Layer 0's weights, drawn once; the other layers hold copies of its experts (other addresses, so no cache reuse)
    # with routers and biases of their own.
    L0 = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=0, zipf=cfg["zipf"])
    ex_bytes = 2 * moe.row_bytes(gt, H) * F + moe.row_bytes(dt, F) * H
    sh_bytes = 2 * moe.row_bytes(sgt, H) * F + moe.row_bytes(sdt, F) * H
    router_bytes = (E + 1) * H * 2
    x = h.tokens(2026, T, H)
    # Layers: enough that the touched bytes (each layer's distinct experts from its own routing, its shared expert and
    # router) pass 512 MB; layer 0's routing (on the CPU) sizes the first estimate.
    _, ids0, _ = L0.oracle_route(x)
    est = len(set(ids0.ravel().tolist())) * ex_bytes + sh_bytes + router_bytes
    n_layer = int(min(64, max(8, np.ceil(600e6 / est))))
    blk = moe.MoeBlock(H, F, E, K, gt, dt, True, sgt, sdt, n_layer=n_layer, max_tokens=16)
    L0.upload(blk, 0)
    for l in range(1, n_layer):
        Ll = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=l, zipf=cfg["zipf"], experts=[],
                     has_shared=False)
        blk.load_router(l, Ll.router, Ll.bias)
        blk.copy_experts(0, l)
    xd, yd, idsd = hip.malloc(x.nbytes), hip.malloc(x.nbytes), hip.malloc(T * K * 4)
    hip.h2d(xd, x)
    # Routing per layer (outside the timed region): distinct experts, for the algorithmic bytes.
    distinct = []
    ids = np.empty((T, K), np.int32)
    for l in range(n_layer):
        blk.forward_async(l, xd, T, yd, idsd)
        hip.sync()
        hip.d2h(ids, idsd)
        distinct.append(len(set(ids.ravel().tolist())))
    touched_all = sum(d * ex_bytes + sh_bytes + router_bytes for d in distinct)
    setup_s = time.time() - t_setup

    for i in range(warmup):
        blk.forward_async(i % n_layer, xd, T, yd)
    blk.check()  # fails the run on a decode wait that gave up (MOE_TIMEOUT)

    def steps_once():
        for i in range(steps):
            blk.forward_async(i % n_layer, xd, T, yd)

    t0, t1, ktimes, nf = timed_steps(hip, blk, steps_once, steps)
    blk.check()
    ms_step = (t1 - t0) * 1e3 / steps
    tok_s = T * steps / (t1 - t0)

    # Algorithmic bytes (the weights of every expert touched, the shared one, the router, once each), per step from
    # that step's layer's routing.
    nd = np.array([distinct[i % n_layer] for i in range(steps)], dtype=np.float64)
    gu_bytes = (nd.mean() * 2 * moe.row_bytes(gt, H) * F + 2 * moe.row_bytes(sgt, H) * F)
    dn_bytes = (nd.mean() * moe.row_bytes(dt, F) * H + moe.row_bytes(sdt, F) * H)
    block_bytes = nd.mean() * ex_bytes + sh_bytes + router_bytes
    k_ms = ktimes.get("moe_decode", float("nan"))
    k_gbs = block_bytes / (k_ms * 1e-3) / 1e9
    block_gbs = block_bytes / (ms_step * 1e-3) / 1e9

    # Parity of this workload (layer 0) against the oracle, and the CPU baseline.
    y = np.empty_like(x)
    blk.forward_async(0, xd, T, yd, idsd)
    hip.sync()
    hip.d2h(y, yd)
    hip.d2h(ids, idsd)
    yo, io, wo = L0.oracle_forward(x, nthreads=16)
    parity = dict(ids_equal=bool(np.array_equal(ids, io)), y_bit_exact=bool(np.array_equal(y, yo)),
                  max_abs=h.max_abs(y, yo), rel_l2=h.rel_l2(y, yo))
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(h, L0, x, block_bytes / T / 1e9, "GB/s", check=y)
    out = {
        "metric": "MoE block tokens/s + achieved HBM GB/s (decode), TFLOP/s (prefill) on 1 GPU",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": cfg["name"], "n_embd": H, "n_ff": F, "n_expert": E, "n_used": K, "shared": True,
                   "tokens": T, "types": [moe.TYPE_NAMES[t] for t in cfg["types"]], "resident_layers": n_layer,
                   "mean_distinct_experts": round(float(nd.mean()), 2),
                   "touched_bytes_all_layers": int(touched_all)},
        "roofline": {"bound": "hbm", "kernel": "moe_decode", "achieved": round(k_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(k_gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(key),
                     "algorithmic_bytes_per_launch": int(block_bytes), "avg_launch_ms": round(k_ms, 5)},
        "block": {"achieved_gbs": round(block_gbs, 1), "frac": round(block_gbs / HBM_PEAK_GBS, 4),
                  "gate_up_bytes": int(gu_bytes), "down_bytes": int(dn_bytes),
                  "kernel_avg_ms": {k: round(v, 5) for k, v in ktimes.items()}, "timed_forwards": nf},
        "parity": parity,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    blk.close()
    return out


def hc(args, cfg, moe, h):
    """The block with its hyper-connection mix and combine (moe_forward_hc_async on the residual streams R, T x 4 x H)
    against the block alone (moe_forward_async) on the same weights: the difference is the mix's and combine's
    kernels. Their roofline is the fp64 matrix cores' (the down GEMM, (lr + 4) x 4H against bf16(n), and the up
    GEMM, 4H x lr against bf16(l), summed exactly in fp64 and certified): the two GEMMs' flops over the whole
    difference, so a lower bound of their rate. Parity: R, y and the ids of a 64-token sample against the oracle's
    mix, block and combine."""
    gt, dt, sgt, sdt = cfg["types"]
    T, lr = cfg["T"], cfg["hc_lr"]
    steps = (50 if T > 16 else 1000) if args.steps is None else args.steps
    warmup = (5 if T > 16 else 100) if args.warmup is None else args.warmup
    hip = Hip()
    t_setup = time.time()
    L = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=0, zipf=cfg["zipf"])
    hm = h.HcModule(H, lr, seed=3)
    blk = moe.MoeBlock(H, F, E, K, gt, dt, True, sgt, sdt, max_tokens=max(T, 16), hc_lr=lr)
    L.upload(blk, 0)
    hm.load(blk, 0)
    R = moe.synth_normal(2026, 4242, T * 4 * H, 1.0).reshape(T, 4, H).astype(np.float32)
    x = h.tokens(2026, T, H)
    Rd, xd, yd = hip.malloc(R.nbytes), hip.malloc(x.nbytes), hip.malloc(x.nbytes)
    hip.h2d(Rd, R)
    hip.h2d(xd, x)
    setup_s = time.time() - t_setup

    def run(fn):
        for _ in range(warmup):
            fn()
        hip.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        hip.sync()
        return (time.perf_counter() - t0) * 1e3 / steps

    blk.check()
    hc_ms = run(lambda: blk.forward_hc_async(0, Rd, T, yd))  # R accumulates its combine step after step
    plain_ms = run(lambda: blk.forward_async(0, xd, T, yd))
    blk.check()
    D = 4 * H
    flop = 2.0 * T * (lr + 4) * D + 2.0 * T * D * lr
    mix_ms = hc_ms - plain_ms
    if T > 16:  # the prefill kernels: fp64 matrix cores
        roof = {"bound": "mfma", "kernel": "pf_hc_gemm (down and up) and the mix's other kernels",
                "achieved": round(flop / (mix_ms * 1e-3) / 1e12, 2), "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(flop / (mix_ms * 1e-3) / 1e12 / FP64_PEAK_TFLOPS, 4), "traffic": None,
                "algorithmic_flop_per_launch": flop, "avg_launch_ms": round(mix_ms, 4)}
    else:  # the decode launch's items: the module's weights read once (bf16 W_down, W_inject, W_up)
        wbytes = 2.0 * ((lr + 4) * D + D * lr)
        roof = {"bound": "hbm", "kernel": "moe_decode's hyper-connection items",
                "achieved": round(wbytes / (mix_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(wbytes / (mix_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                "algorithmic_bytes_per_launch": int(wbytes), "avg_launch_ms": round(mix_ms, 4)}
    n = min(64, T)
    Rs = R[:n]
    Rg, yg, ig, _ = blk.forward_hc(0, Rs)
    xo, inj = hm.pre(Rs)
    yo, io, _ = L.oracle_forward(xo, nthreads=16)
    Ro = hm.post(Rs, inj, yo)
    parity = dict(sample_tokens=n, ids_equal=bool(np.array_equal(ig, io)), R_bit_exact=bool(np.array_equal(Rg, Ro)),
                  R_max_abs=h.max_abs(Rg, Ro), R_rel_l2=h.rel_l2(Rg, Ro), y_max_abs=h.max_abs(yg, yo),
                  y_rel_l2=h.rel_l2(yg, yo))
    out = {
        "metric": "MoE block with hyper-connection mix and combine, tokens/s (not a BASELINE metric)",
        "value": round(T / (hc_ms * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(hc_ms, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f64", "data": "synthetic",
        "config": {"workload": cfg["name"], "n_embd": H, "n_ff": F, "n_expert": E, "n_used": K, "shared": True,
                   "tokens": T, "hc_lr": lr, "types": [moe.TYPE_NAMES[t] for t in cfg["types"]]},
        "roofline": roof,
        "block": {"block_alone_ms": round(plain_ms, 4), "mix_and_combine_ms": round(mix_ms, 4)},
        "parity": parity,
        "cpu_baseline": None,
        "setup_s": round(setup_s, 1),
    }
    blk.close()
    print(json.dumps(out), flush=True)


def stack(args, cfg, moe, h):
    """Config 5: the model's 48 MoE blocks in sequence (attention and DeltaNet omitted). With those omitted there is no
    residual stream to keep the activations RMSNorm-like, so every block takes the step's synthetic tokens (N(0, 1),
    as at the configs' block input) and the blocks run one after another on one stream; chaining the raw block
    outputs instead would shrink them layer by layer and collapse the routing onto a few experts. The layers have
    their own routers and Zipf biases; their experts are device copies of layer 0's (other addresses, so every
    layer's weights are read from HBM: 48 x 763 MB resident). A step is one token (decode) or 4096 tokens in two
    chunks of 2048 (prefill) through all 48 layers."""
    gt, dt, sgt, sdt = cfg["types"]
    NL, T = cfg["layers"], cfg["T"]
    chunk = cfg.get("chunk", T)
    decode = T <= 16
    steps = (200 if decode else 3) if args.steps is None else args.steps
    warmup = (20 if decode else 1) if args.warmup is None else args.warmup
    hip = Hip()
    t_setup = time.time()
    L0 = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=0, zipf=cfg["zipf"])
    blk = moe.MoeBlock(H, F, E, K, gt, dt, True, sgt, sdt, n_layer=NL, max_tokens=chunk)
    L0.upload(blk, 0)
    layers = [L0]
    for l in range(1, NL):
        Ll = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=l, zipf=cfg["zipf"], experts=[], has_shared=False)
        blk.load_router(l, Ll.router, Ll.bias)
        blk.copy_experts(0, l)
        Ll.experts, Ll.shared, Ll.has_shared = L0.experts, L0.shared, True  # the oracle's view of the copies
        layers.append(Ll)
    x = h.tokens(2026, T, H)
    bufs = [hip.malloc(chunk * H * 4), hip.malloc(chunk * H * 4)]
    idsd = hip.malloc(chunk * K * 4)

    xdev = hip.malloc(T * H * 4)
    hip.h2d(xdev, x)

    def run(c0, n, collect=None):
        xc = C.c_void_p(xdev.value + c0 * H * 4)
        for l in range(NL):
            blk.forward_async(l, xc, n, bufs[l % 2], idsd if collect is not None else None)
            if collect is not None:
                hip.sync()
                ids = np.empty((n, K), np.int32)
                hip.d2h(ids, idsd)
                collect.append(len(set(ids.ravel().tolist())))

    distinct = []
    run(0, min(chunk, T), distinct)
    hip.sync()
    setup_s = time.time() - t_setup
    for _ in range(warmup):
        for c0 in range(0, T, chunk):
            run(c0, min(chunk, T - c0))
    hip.sync()
    def steps_once():
        for _ in range(steps):
            for c0 in range(0, T, chunk):
                run(c0, min(chunk, T - c0))

    blk.check()
    if decode:
        t0, t1, ktimes, nf = timed_steps(hip, blk, steps_once, steps * NL)
    else:
        t0, t1, ktimes, nf = timed_steps_per_launch(hip, blk, steps_once)
    blk.check()
    ms_step = (t1 - t0) * 1e3 / steps
    tok_s = T * steps / (t1 - t0)
    ex_bytes = 2 * moe.row_bytes(gt, H) * F + moe.row_bytes(dt, F) * H
    sh_bytes = 2 * moe.row_bytes(sgt, H) * F + moe.row_bytes(sdt, F) * H
    router_bytes = (E + 1) * H * 2
    layer_bytes = np.mean(distinct) * ex_bytes + sh_bytes + router_bytes  # per layer (first chunk's routing)
    # Parity: the oracle through the same 48 layers, on a sample of the tokens.
    sample = np.r_[0:min(T, 4)] if decode else np.r_[0:4, chunk:chunk + 4]
    y = np.empty((chunk, H), np.float32)
    outs = []
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        run(c0, n)
        hip.sync()
        yy = np.empty((n, H), np.float32)
        hip.d2h(yy, bufs[(NL - 1) % 2])
        outs.append(yy)
    yall = np.concatenate(outs)

    def oracle_stack(smp):
        t0_ = time.perf_counter()
        for l in range(NL):  # the CPU does every layer too; the last layer's output is compared
            xo_, _, _ = layers[l].oracle_forward(x[smp], nthreads=min(16, os.cpu_count() or 1))
        return xo_, time.perf_counter() - t0_

    xo, cpu_s = oracle_stack(sample)
    if not args.no_cpu and not decode:  # prefill: as many tokens as --cpu-seconds allows, from both chunks
        per = max(4, int(len(sample) * args.cpu_seconds / max(cpu_s, 1e-6)) // 2)
        if 2 * per > len(sample):
            sample = np.r_[0:min(per, chunk), chunk:chunk + min(per, T - chunk)]
            xo, cpu_s = oracle_stack(sample)
    yg = yall[sample]
    parity = dict(sample_tokens=len(sample), y_bit_exact=bool(np.array_equal(yg, xo)), max_abs=h.max_abs(yg, xo),
                  rel_l2=h.rel_l2(yg, xo))
    cores = min(16, os.cpu_count() or 1)
    cpu = None if args.no_cpu else {
        "value": round(len(sample) / cpu_s, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
        "sample": "%d tokens through the 48 layers by oracle/oracle.c with %d OpenMP threads, %.1f s"
                  % (len(sample), cores, cpu_s)}
    if decode:
        k_ms = ktimes.get("moe_decode", float("nan"))
        roof = {"bound": "hbm", "kernel": "moe_decode", "achieved": round(layer_bytes / (k_ms * 1e-3) / 1e9, 1),
                "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(layer_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                "traffic": None, "algorithmic_bytes_per_launch": int(layer_bytes), "avg_launch_ms": round(k_ms, 5)}
    else:
        # The routed gate/up launch (the shared expert's runs beside the router on a second stream).
        gu_ms = ktimes.get("pf_gate_up", float("nan"))
        gu_flop = 2.0 * (chunk * K) * 2 * F * H
        roof = {"bound": "mfma", "kernel": GU_KERNEL.get(cfg["types"][0], "pf_gemm16"),
                "achieved": round(gu_flop / (gu_ms * 1e-3) / 1e12, 2),
                "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                "frac": round(gu_flop / (gu_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
                "traffic": measured_prefill_traffic(args.config),
                "algorithmic_flop_per_launch": gu_flop, "avg_launch_ms": round(gu_ms, 4)}
    out = {
        "metric": "MoE block tokens/s + achieved HBM GB/s (decode), TFLOP/s (prefill) on 1 GPU",
        "value": round(tok_s, 2), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": cfg["name"], "layers": NL, "n_embd": H, "n_ff": F, "n_expert": E, "n_used": K,
                   "tokens": T, "chunk": chunk, "types": [moe.TYPE_NAMES[t] for t in cfg["types"]],
                   "mean_distinct_experts_per_layer": round(float(np.mean(distinct)), 2)},
        "roofline": roof,
        "block": {"stack_hbm_gbs": round(NL * layer_bytes * (T // chunk if not decode else 1) / (ms_step * 1e-3) / 1e9, 1)
                  if decode else None,
                  "kernel_avg_ms": {k: round(v, 5) for k, v in ktimes.items()}, "timed_forwards": nf},
        "parity": parity,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    print(json.dumps(out), flush=True)
    blk.close()


def prefill(args, cfg, key, moe, h):
    """Config 4: one forward of 2048 tokens is a step. One resident layer: its 906 MB of experts already exceed the
    Infinity Cache, and every step reads all of them."""
    steps = 100 if args.steps is None else args.steps
    warmup = 10 if args.warmup is None else args.warmup
    gt, dt, sgt, sdt = cfg["types"]
    T = cfg["T"]
    hip = Hip()
    t_setup = time.time()
    L0 = h.Layer(H, F, E, K, gt, dt, sgt, sdt, seed=2026, layer=0, zipf=cfg["zipf"])
    blk = moe.MoeBlock(H, F, E, K, gt, dt, True, sgt, sdt, n_layer=1, max_tokens=T)
    L0.upload(blk, 0)
    x = h.tokens(2026, T, H)
    xd, yd, idsd = hip.malloc(x.nbytes), hip.malloc(x.nbytes), hip.malloc(T * K * 4)
    hip.h2d(xd, x)
    ids = np.empty((T, K), np.int32)
    blk.forward_async(0, xd, T, yd, idsd)
    hip.sync()
    hip.d2h(ids, idsd)
    touched = len(set(ids.ravel().tolist()))
    setup_s = time.time() - t_setup
    for _ in range(warmup):
        blk.forward_async(0, xd, T, yd)
    blk.check()

    def steps_once():
        for _ in range(steps):
            blk.forward_async(0, xd, T, yd)

    t0, t1, ktimes, nf = timed_steps_per_launch(hip, blk, steps_once)
    blk.check()
    ms_step = (t1 - t0) * 1e3 / steps
    tok_s = T * steps / (t1 - t0)
    # Algorithmic work: 2 FLOP per weight per assignment (gate, up, down), the shared expert per token, the router's
    # (E + 1) rows per token; bytes: every touched expert's weights, the shared one, the router, once.
    ex_bytes = 2 * moe.row_bytes(gt, H) * F + moe.row_bytes(dt, F) * H
    sh_bytes = 2 * moe.row_bytes(sgt, H) * F + moe.row_bytes(sdt, F) * H
    gu_flop = 2.0 * (T * K + T) * 2 * F * H
    dn_flop = 2.0 * (T * K + T) * F * H
    router_flop = 2.0 * T * (E + 1) * H
    block_flop = gu_flop + dn_flop + router_flop
    block_bytes = touched * ex_bytes + sh_bytes + (E + 1) * H * 2
    # The roofline's kernel is the routed gate/up launch, on its own FLOPs (the shared expert's launch runs beside the
    # router on a second stream, overlapped, so the two durations do not add up to the time they take).
    gu_ms = ktimes.get("pf_gate_up", float("nan"))
    gu_routed_flop = 2.0 * (T * K) * 2 * F * H
    gu_tops = gu_routed_flop / (gu_ms * 1e-3) / 1e12
    # Parity on a sample of tokens (each token's output depends on that token alone): ids and w on all tokens, y on
    # the sample, against the oracle.
    y = np.empty_like(x)
    w = np.empty((T, K), np.float32)
    wd = hip.malloc(T * K * 4)
    blk.prefill_exact_tokens()  # clears the count: the next forward's alone is reported
    blk.forward_async(0, xd, T, yd, idsd, wd)
    hip.sync()
    hip.d2h(y, yd)
    hip.d2h(ids, idsd)
    hip.d2h(w, wd)
    _, io, wo = L0.oracle_route(x)
    sample = np.r_[0:64, T // 2:T // 2 + 64, T - 64:T]
    yo, _, _ = L0.oracle_forward(x[sample], nthreads=min(16, os.cpu_count() or 1))
    ma, rl = h.max_abs(y[sample], yo), h.rel_l2(y[sample], yo)
    parity = dict(sample_tokens=len(sample), ids_equal_all_tokens=bool(np.array_equal(ids, io)),
                  w_bit_exact_all_tokens=bool(np.array_equal(w, wo)), w_max_abs_all_tokens=h.max_abs(w, wo),
                  y_bit_exact=bool(np.array_equal(y[sample], yo)), max_abs=ma, rel_l2=rl,
                  y_within_tolerance=bool(ma <= h.TOL_ABS and rl <= h.TOL_REL),
                  router="matrix-core, certified top-k", exact_sum_tokens=blk.prefill_exact_tokens())
    cpu = None
    if not args.no_cpu:  # a bounded sample: 192 of the chunk's tokens (all cores), 32 (one core)
        cpu = cpu_baseline(h, L0, x[sample], block_flop / T / 1e12, "TFLOP/s", check=y[sample], one_core_tokens=32)
    out = {
        "metric": "MoE block tokens/s + achieved HBM GB/s (decode), TFLOP/s (prefill) on 1 GPU",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": cfg["name"], "n_embd": H, "n_ff": F, "n_expert": E, "n_used": K, "shared": True,
                   "tokens": T, "types": [moe.TYPE_NAMES[t] for t in cfg["types"]], "touched_experts": touched},
        "roofline": {"bound": "mfma", "kernel": GU_KERNEL.get(cfg["types"][0], "pf_gemm16"), "achieved": round(gu_tops, 2),
                     "peak": INT8_PEAK_TOPS,
                     "unit": "TFLOP/s", "frac": round(gu_tops / INT8_PEAK_TOPS, 4),
                     "traffic": measured_prefill_traffic(key),
                     "algorithmic_flop_per_launch": gu_routed_flop, "avg_launch_ms": round(gu_ms, 4)},
        "block": {"tflops": round(block_flop / (ms_step * 1e-3) / 1e12, 2),
                  "hbm_gbs": round(block_bytes / (ms_step * 1e-3) / 1e9, 1),
                  "hbm_frac": round(block_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                  "algorithmic_flop": block_flop, "algorithmic_bytes": block_bytes,
                  "kernel_avg_ms": {k: round(v, 4) for k, v in ktimes.items()}, "timed_forwards": nf},
        "parity": parity,
        "cpu_baseline": cpu,
        "setup_s": round(setup_s, 1),
    }
    blk.close()
    return out


if __name__ == "__main__":
    main()
