"""Benchmark of the sageattn_vc hot path on one MI355X (BASELINE.json metric).

A step is one pass of the hot path over one batch: preprocessing (K centring,
Sage INT8 Q/K, V E4M3 [+ grouping and block smoothing]) followed by the fused
attention kernel, with bf16 inputs already resident in HBM. The headline value
is the fused kernel's effective TOPS = 4*B*H*Nq*Nk*D / kernel time, timed with
HIP events on the stream the kernels run on; preprocessing is timed separately.

    python bench.py [--steps K] [--warmup W] [--config main|smooth|d64|long|cpu] [--qk int8|fp8]

--qk fp8 measures the block-scaled FP8 QK variant (the reference's experimental vc27:
E4M3 Q/K in 64/128-row blocks, K centred in binary32) on the same workload; it has no
V smoothing, so it runs the configurations without smoothing only.

Prints ONE JSON line (rank 0, N=1). --gpus N with N > 1 exits: this build runs
on one GPU only.
"""
import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cake-opt-vc_attention_amd"))
sys.path.insert(0, str(ROOT))

PEAK_TOPS = 5000.0      # MI355X dense INT8 / FP8 MFMA, TOPS (published)
PEAK_CLOCK_GHZ = 2.4    # engine clock of the published peak (256 CUs x 4 SIMDs x 2048 ops/clock)
PEAK_HBM_GBS = 8000.0   # MI355X HBM3E, GB/s (published)

# HBM bytes per fused-kernel launch, measured with rocprofv3 --pmc FETCH_SIZE (scaled by
# 2.0, the factor a plain 1 GiB copy reads) plus WRITE_SIZE (factor 1.0); the runs and their
# commands are in profiles/attn_kernel_<config>_hbm_bytes.txt (FP8 QK variant:
# profiles/attn_kernel_fp8_main_hbm_bytes.txt). Counters cannot be read from inside this
# process, so the figure is keyed by QK format and configuration and null where unmeasured.
MEASURED_TRAFFIC_BYTES = {("int8", "main"): 3.174e9, ("int8", "d64"): 1.769e9, ("int8", "smooth"): 3.133e9,
                          ("int8", "long"): 1.1465e10, ("fp8", "main"): 3.133e9}
# VALU instructions per wave and 128-key tile of the fused kernel ((SQ_INSTS_VALU -
# SQ_INSTS_MFMA) / (waves x tiles), rocprofv3 --pmc; profiles/attn_kernel_<config>_counters.txt),
# and the best issue rate measured for the kernel's
# per-score VALU chain with two waves per SIMD (3.0 cycles per instruction per SIMD,
# register-only microbenchmark). Together they give the VALU issue bound of a launch.
MEASURED_VALU_PER_WAVE_TILE = {("int8", "main"): 261.1, ("int8", "d64"): 386.1, ("int8", "smooth"): 395.4,
                               ("int8", "long"): 385.3}
VALU_CYCLES_PER_INSTR = 3.0
SIMDS = 1024            # 256 CUs x 4 SIMDs

CONFIGS = {
    # name: (B, H, N, D, kind, v_smooth, description)
    "main": (1, 28, 37741, 128, "normal", False,
             "BNSD [1,28,37741,128] bf16, Q/K/V N(0,1) seed 0, non-causal, sm_scale=1/sqrt(128), "
             "INT8 QK (Sage per-thread scales) + ExpCast FP8 E4M3 PV, V smoothing off"),
    "smooth": (1, 28, 37741, 128, "outlier", True,
               "BNSD [1,28,37741,128] bf16, K outlier channels, clustered V; ExpCast + V grouping "
               "(8 clusters, 2 Lloyd iterations) + 128-token block-mean smoothing"),
    "d64": (1, 40, 32760, 64, "normal", True,
            "BNSD [1,40,32760,64] bf16, N(0,1); ExpCast + V smoothing"),
    "long": (1, 28, 75482, 128, "student", True,
             "BNSD [1,28,75482,128] bf16, Q,K 0.5*Student-t(4), V N(0,1); full pipeline"),
    "cpu": (1, 2, 2048, 128, "normal", False,
            "BNSD [1,2,2048,128] bf16 N(0,1), smoothing off (the reference's CPU plumbing case)"),
}


def make_inputs(B, H, N, D, kind, seed=0):
    """Seeded CPU generation (q, then k, then v), cast to bf16."""
    import numpy as np
    import torch
    g = torch.Generator().manual_seed(seed)
    if kind == "normal":
        q = torch.randn(B, H, N, D, generator=g)
        k = torch.randn(B, H, N, D, generator=g)
        v = torch.randn(B, H, N, D, generator=g)
    elif kind == "outlier":
        q = torch.randn(B, H, N, D, generator=g)
        k = torch.randn(B, H, N, D, generator=g) + torch.randn(B, H, 1, D, generator=g) * 2.0
        cent = torch.randn(B, H, 8, D, generator=g) * 2.0 ** 0.5
        assign = torch.randint(0, 8, (B, H, N), generator=g)
        v = torch.gather(cent, 2, assign[..., None].expand(B, H, N, D)) + torch.randn(B, H, N, D, generator=g) * 0.3 ** 0.5
    elif kind == "student":
        rng = np.random.Generator(np.random.PCG64(seed))
        q = torch.from_numpy(0.5 * rng.standard_t(4, size=(B, H, N, D)).astype(np.float32))
        k = torch.from_numpy(0.5 * rng.standard_t(4, size=(B, H, N, D)).astype(np.float32))
        v = torch.randn(B, H, N, D, generator=g)
    else:
        raise ValueError(kind)
    return q.to(torch.bfloat16), k.to(torch.bfloat16), v.to(torch.bfloat16)


def cpu_baseline(q, k, v, smooth, rows, budget_s, qk="int8", rotate=False):
    """The CPU oracle (C restatement, OpenMP over rows) on the box's host cores:
    full preprocessing of the same workload plus attention for `rows` evenly
    spaced query rows of every head against all keys, extrapolated to all rows."""
    import numpy as np
    import torch
    from oracle import vc_oracle as o

    bits = lambda x: x.contiguous().view(torch.int16).numpy().view(np.uint16)
    B, H, N, D = q.shape
    qb, kb, vb = bits(q), bits(k), bits(v)
    t0 = time.perf_counter()
    st = o.prepare_fp8(qb, kb, vb) if qk == "fp8" else o.prepare(qb, kb, vb, v_smooth=smooth, qk_hadamard=rotate)
    prep_s = time.perf_counter() - t0
    # Without smoothing the GPU path uses the folded ExpCast encode, whose fallback is decided
    # per 16-row group: sample whole groups so the oracle's group pass covers only them.
    affine = not smooth
    if affine:
        starts = o.query_indices((N + 15) // 16, max(1, rows // 16)) * 16
        ids = np.unique(np.clip((starts[:, None] + np.arange(16)).ravel(), 0, N - 1))
    else:
        ids = o.query_indices(N, rows)
    t0 = time.perf_counter()
    o.reference(st, query_indices=ids, affine=affine)
    attn_s = time.perf_counter() - t0
    ops = 4.0 * B * H * len(ids) * N * D
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    full_s = prep_s + attn_s * N / len(ids)
    return {
        "value": ops / attn_s / 1e12,
        "unit": "TOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"oracle/vc_oracle.c: attention of {len(ids)} query rows "
                  f"({'evenly spaced 16-row groups, folded ExpCast encode' if affine else 'evenly spaced, ExpCast'}"
                  f"{', FP8 block QK' if qk == 'fp8' else ''}) "
                  f"x all {N} keys x {B * H} heads (P bytes + decoded-payload fp64 accumulation), OpenMP over rows; "
                  f"value = 4*B*H*rows*N*D / time. Full preprocessing of the same inputs (OpenMP over heads and channels) "
                  f"took {prep_s:.2f} s; extrapolated full forward = {full_s:.1f} s",
        "attention_s": attn_s,
        "prep_s": prep_s,
        "sample_rows_per_head": int(len(ids)),
        "extrapolated_full_forward_s": full_s,
        "extrapolation": "linear in query rows (attention) + full preprocessing",
        "cpu_model": cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "omp_threads": threads,
        "torch_threads": torch.get_num_threads(),
    }


class PowerSampler:
    """Board telemetry beside a launch loop (amdsmi, the library behind amd-smi): socket power,
    per-XCD engine clocks, GFX rail voltage and temperatures every `period` seconds, and the
    firmware's throttle-residency accumulators read at start and stop, which say what held
    the clock below its maximum: PPT (package power), socket / VR / HBM thermal or PROCHOT.
    Residency = delta of a reason's accumulator / delta of accumulation_counter."""

    REASONS = ("ppt_residency_acc", "socket_thm_residency_acc", "vr_thm_residency_acc",
               "hbm_thm_residency_acc", "prochot_residency_acc")

    def __init__(self, torch_device, period=0.25):
        import threading
        import amdsmi
        self.smi = amdsmi
        amdsmi.amdsmi_init(amdsmi.AmdSmiInitFlags.INIT_AMD_GPUS)
        handles = amdsmi.amdsmi_get_processor_handles()
        self.handle = handles[0]
        try:  # the handle whose PCI bus matches the torch device (a box may list more GPUs)
            import torch
            bus = torch.cuda.get_device_properties(torch_device).pci_bus_id
            for h in handles:
                if int(amdsmi.amdsmi_get_gpu_device_bdf(h).split(":")[1], 16) == bus:
                    self.handle = h
        except Exception:
            pass
        self.period, self.samples, self.stop_ev = period, [], threading.Event()
        self.thread = threading.Thread(target=self._run, daemon=True)

    def _metrics(self):
        return self.smi.amdsmi_get_gpu_metrics_info(self.handle)

    def _run(self):
        while not self.stop_ev.wait(self.period):
            m = self._metrics()
            self.samples.append({k: m.get(k) for k in ("current_socket_power", "current_gfxclks", "voltage_gfx",
                                                        "temperature_hotspot", "temperature_vrgfx",
                                                        "throttle_status", "indep_throttle_status")})

    def start(self):
        self.t0, self.m0 = time.perf_counter(), self._metrics()
        self.thread.start()
        return self

    def stop(self):
        self.stop_ev.set()
        self.thread.join()
        m1, t1 = self._metrics(), time.perf_counter()
        num = lambda x: x if isinstance(x, (int, float)) else None
        dacc = (num(m1.get("accumulation_counter")) or 0) - (num(self.m0.get("accumulation_counter")) or 0)
        residency = {}
        for r in self.REASONS:
            a, b = num(self.m0.get(r)), num(m1.get(r))
            residency[r.replace("_residency_acc", "")] = round((b - a) / dacc, 4) if dacc > 0 and a is not None and b is not None else None
        s = [x for x in self.samples if isinstance(x["current_socket_power"], (int, float))]
        mean = lambda xs: round(sum(xs) / len(xs), 1) if xs else None
        clocks = [x["current_gfxclks"] for x in s if isinstance(x["current_gfxclks"], list)]
        xcd = [mean([c[i] for c in clocks if isinstance(c[i], (int, float))]) for i in range(8)] if clocks else None
        caps = {}
        for ind, name in ((0, "ppt0"), (1, "ppt1")):
            try:
                ci = self.smi.amdsmi_get_power_cap_info(self.handle, ind)
                caps[name] = {k: ci[k] / 1e6 if isinstance(ci[k], (int, float)) else ci[k] for k in ("power_cap", "default_power_cap", "max_power_cap")}
            except Exception as e:  # a sensor the board does not have
                caps[name] = str(e)[:80]
        return {"window_s": round(t1 - self.t0, 2), "samples": len(s),
                "socket_power_w_mean": mean([x["current_socket_power"] for x in s]),
                "socket_power_w_max": max((x["current_socket_power"] for x in s), default=None),
                "gfxclk_mhz_per_xcd_mean": xcd,
                "voltage_gfx_mv_mean": mean([x["voltage_gfx"] for x in s if isinstance(x["voltage_gfx"], (int, float))]),
                "temperature_hotspot_c_max": max((x["temperature_hotspot"] for x in s if isinstance(x["temperature_hotspot"], (int, float))), default=None),
                "temperature_vrgfx_c_max": max((x["temperature_vrgfx"] for x in s if isinstance(x["temperature_vrgfx"], (int, float))), default=None),
                "throttle_status_seen": sorted({str(x["throttle_status"]) for x in s}),
                "indep_throttle_status_seen": sorted({str(x["indep_throttle_status"]) for x in s}),
                "throttle_residency": residency, "accumulation_ticks": dacc, "power_caps_w": caps}


def cpu_model():
    """CPU model name from /proc/cpuinfo (platform.processor() is empty on the GPU box)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="main", choices=sorted(CONFIGS))
    ap.add_argument("--cpu-rows", type=int, default=2048, help="query rows per head for the CPU baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-clock", action="store_true",
                    help="skip the engine-clock burst after the timed steps (for kernel-trace profiles)")
    ap.add_argument("--qk-hadamard", action="store_true",
                    help="rotate Q and the centred K (normalized Hadamard) inside the INT8 quantizers")
    ap.add_argument("--qk", default="int8", choices=("int8", "fp8"),
                    help="int8: the sageattn_vc path (headline); fp8: the block-scaled FP8 QK variant")
    ap.add_argument("--mode", default="full", choices=("full", "kernel", "copy"),
                    help="full: the benchmark; kernel: prepare once, then only the fused kernel "
                         "(--steps launches, for profilers); copy: a plain 1 GiB device copy "
                         "(calibrates profiler byte counters)")
    ap.add_argument("--ready-file", default=None,
                    help="kernel mode: create this file when the launch loop starts (a power or clock "
                         "sampler running beside the benchmark waits for it)")
    ap.add_argument("--power", action="store_true",
                    help="kernel mode: sample board power, engine clocks and the firmware's throttle "
                         "residency (amdsmi) over the timed launches")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs the sageattn_vc path on ONE GPU; multi-GPU runs are not part of it "
              "(the path would shard by (batch, head) with no communication).", file=sys.stderr)
        sys.exit(2)

    import torch
    import vcx

    B, H, N, D, kind, smooth, desc = CONFIGS[args.config]
    fp8 = args.qk == "fp8"
    if fp8 and args.qk_hadamard:
        print("bench.py: --qk-hadamard applies to the INT8 path", file=sys.stderr)
        sys.exit(2)
    if fp8 and smooth:
        print(f"bench.py: --qk fp8 has no V smoothing; config {args.config!r} needs it", file=sys.stderr)
        sys.exit(2)
    if fp8:
        desc = desc.replace("INT8 QK (Sage per-thread scales)", "FP8 E4M3 QK (64/128-row block scales, K centred)")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.mode == "copy":
        src = torch.ones(1 << 29, dtype=torch.int16, device=dev)  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"mode": "copy", "bytes_read_per_launch": src.numel() * 2,
                          "bytes_written_per_launch": dst.numel() * 2, "launches": max(args.steps, 1)}))
        return
    qc, kc, vc_ = make_inputs(B, H, N, D, kind)
    q, k, v = (x.to(dev) for x in (qc, kc, vc_))
    scale = D ** -0.5
    clusters, iterations = 8, 2

    def prep():
        if fp8:
            q8, qs, k8, ks, _ = vcx.prepare_qk_fp8(q, k)
            v8, vs, means = vcx.prepare_v(v, None, smooth=False, channel_scale=True)
            return q8, qs, k8, ks, v8, vs, means
        perm = vcx.group_values(v, clusters, iterations) if smooth else None
        q8, qs, k8, ks, _ = vcx.prepare_qk(q, k, perm, hadamard=args.qk_hadamard)
        v8, vs, means = vcx.prepare_v(v, perm, smooth=smooth, channel_scale=True)
        return q8, qs, k8, ks, v8, vs, means

    out = torch.empty((B, H, N, D), dtype=torch.bfloat16, device=dev)

    def fused(p):
        q8, qs, k8, ks, v8, vs, means = p
        if fp8:  # the reference's FP8 kernel folds the ExpCast encode
            vcx.forward_fp8(q8, k8, v8, qs, ks, vs, True, 1, scale, affine=True, out=out)
            return
        # the reference's default kernel mode: folded ExpCast encode without block values
        vcx.forward(q8, k8, v8, qs, ks, vs, means, True, smooth, 1, scale, affine=not smooth, out=out)

    if args.mode == "kernel":
        p = prep()
        torch.cuda.synchronize()
        if args.ready_file:
            Path(args.ready_file).write_text("launching\n")
        for _ in range(args.warmup):
            fused(p)
        torch.cuda.synchronize()
        sampler = PowerSampler(dev).start() if args.power else None
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fused(p)
        torch.cuda.synchronize()
        res = {"mode": "kernel", "launches": args.warmup + args.steps, "config": args.config,
               "ms_per_timed_launch": round((time.perf_counter() - t0) * 1e3 / max(args.steps, 1), 4)}
        if sampler is not None:
            res["power"] = sampler.stop()
        print(json.dumps(res), flush=True)
        return
    for _ in range(args.warmup):
        fused(prep())
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record()
        p = prep()
        e1.record()
        fused(p)
        e2.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    prep_ms = sorted(e0.elapsed_time(e1) for e0, e1, _ in ev)
    kern_ms = sorted(e1.elapsed_time(e2) for _, e1, e2 in ev)
    med = lambda xs: xs[len(xs) // 2]
    kernel_ms, prep_med = med(kern_ms), med(prep_ms)
    ops = 4.0 * B * H * N * N * D
    tops = ops / (kernel_ms * 1e-3) / 1e12
    mean_kernel_ms = sum(kern_ms) / len(kern_ms)
    achieved = ops / (mean_kernel_ms * 1e-3) / 1e12
    tiles = (N + 127) // 128
    if fp8:  # block scales: one per 64 query rows and one per key tile, plus the fp32 K mean
        prep_bytes = 9.0 * B * H * N * D + 4.0 * B * H * ((N + 63) // 64 + tiles) + 8.0 * B * H * D
    else:
        prep_bytes = 6.0 * B * H * N * D + 3.0 * B * H * N * D + 4.0 * B * H * ((N + 63) // 64 * 32) \
            + 4.0 * B * H * tiles * 4 + 4.0 * B * H * D + (2.0 * B * H * tiles * D if smooth else 0.0)
    prep_gbs = prep_bytes / (prep_med * 1e-3) / 1e9
    result = {
        "metric": ("sageattn_vc_fp8 (FP8 block QK) " if fp8 else "sageattn_vc ")
                  + f"fused-kernel TOPS at BNSD [{B},{H},{N},{D}] bf16 (4*B*H*N^2*D / kernel time); "
                  "kernel ms and fraction of INT8/FP8 MFMA peak",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("fp8-e4m3" if fp8 else "int8") + " QK / fp8-e4m3 PV, fp32 accumulate",
        "data": "synthetic (seeded torch.Generator on CPU, cast to bf16, copied to HBM before timing)",
        "config": {"workload": desc, "shape_bnsd": [B, H, N, D], "config_name": args.config,
                   "v_smooth": smooth, "expcast": True, "qk_format": "fp8_block" if fp8 else "int8",
                   "qk_hadamard": args.qk_hadamard,
                   "expcast_encode": "unfused (block values)" if smooth else "folded (the reference's default kernel mode)"},
        "kernel_ms": round(kernel_ms, 4),
        "prep_ms": round(prep_med, 4),
        "step_tops": round(ops / (wall_ms * 1e-3) / 1e12, 2),
        "frac_of_mfma_peak": round(tops / PEAK_TOPS, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_TOPS, 4),
                     "traffic": MEASURED_TRAFFIC_BYTES.get((args.qk, args.config)),
                     "kernel": "attn_kernel (fused QK/ExpCast/PV)", "ops_per_launch": ops},
        "roofline_prep": {"bound": "hbm", "achieved": round(prep_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(prep_gbs / PEAK_HBM_GBS, 4), "algorithmic_bytes": prep_bytes},
    }
    # Engine clock, outside the timed region: a short burst of untimed steps right after the
    # timed ones (the GPU still in its sustained state), with probe waves on a second stream
    # over the first 60 % of the fused launches 2..5, then the probe alone with the GPU idle.
    if not args.no_clock:
        side = torch.cuda.Stream(device=dev)
        window_us = max(int(kernel_ms * 600), 100)
        probes = []
        for i in range(5):
            p = prep()
            if i > 0:
                side.wait_stream(torch.cuda.current_stream(dev))
                with torch.cuda.stream(side):
                    probes.append(vcx.clock_probe(window_us, dev))
            fused(p)
        torch.cuda.synchronize()
        per_launch = [pr.ghz() for pr in probes]
        per_wave = [g for pr in probes for g in pr.ghz_per_block()]
        idle_ghz = vcx.clock_probe(2000, dev).ghz()
        load_ghz = sum(per_launch) / len(per_launch)
        result["clock"] = {"engine_ghz_under_load": round(load_ghz, 3), "engine_ghz_idle": round(idle_ghz, 3),
                           "engine_ghz_per_probed_launch": [round(g, 3) for g in per_launch],
                           "engine_ghz_probe_wave_range": [round(min(per_wave), 3), round(max(per_wave), 3)],
                           "peak_basis_ghz": PEAK_CLOCK_GHZ,
                           "frac_at_measured_clock": round(achieved / (PEAK_TOPS * load_ghz / PEAK_CLOCK_GHZ), 4),
                           "method": "s_memtime / s_memrealtime ticks of 8 one-wave probe blocks (one per XCD) on a "
                                     "second stream over the first 60 % of fused launches 2-5 of an untimed burst "
                                     "that follows the timed steps (vcx_clock_probe)"}
    valu = MEASURED_VALU_PER_WAVE_TILE.get((args.qk, args.config))
    if valu is not None:
        # one wave per 32 query rows, every wave walks every key tile
        instr = valu * (B * H * tiles * 4) * tiles
        ghz = result["clock"]["engine_ghz_under_load"] if "clock" in result else PEAK_CLOCK_GHZ
        bound_ms = instr * VALU_CYCLES_PER_INSTR / SIMDS / (ghz * 1e9) * 1e3
        result["roofline_valu"] = {"bound": "valu", "instructions_per_launch": instr,
                                   "cycles_per_instruction": VALU_CYCLES_PER_INSTR, "clock_ghz": ghz,
                                   "bound_ms": round(bound_ms, 4), "frac": round(bound_ms / mean_kernel_ms, 4),
                                   "note": "VALU issue bound of the fused kernel: measured VALU instructions "
                                           "per wave-tile x waves x tiles at the best measured two-wave issue "
                                           "rate; frac = bound / mean kernel time"}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(qc, kc, vc_, smooth, args.cpu_rows, 30.0, args.qk,
                                              args.qk_hadamard)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
