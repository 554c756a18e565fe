"""Benchmark of the bev-kernels hot paths on one MI355X.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--warm] [--no-configs]
                  [--no-cpu-baseline] [--only NAME] [--settle-ms MS]

Prints ONE JSON line. The headline ("step") is one MSDA forward at the BEVFormer
spatial-cross-attention shape (6 cameras, 4 levels, Len_in 30825,
Len_q 10000, 8 heads x 32, 8 points), fp32, with inputs resident in HBM:
  value      algorithmic GB/s = compulsory bytes (value + sampling_loc + attn_weight
             read once, output written once: 435.15 MB) / mean kernel time
  roofline   the same figure against 8 TB/s, kernel time from HIP events on the stream
             the kernel runs on; `traffic` from the committed rocprofv3 counter summary
  secondary  the fused NHWC DCNv2 res4 fp16 forward in MFMA TFLOP/s (2*M*K*Cout flops),
             timed like a configs row (>= 100 launches; mean and median); the configs
             row of that kernel reports these same launches
  configs    every BASELINE configuration x dtype: us, GB/s or TFLOP/s, roofline fraction;
             the backward kernels (MSDA backward, DCN NHWC column-to-image) in GB/s of
             compulsory bytes
  cpu_baseline  the CPU oracle (grid_sample form) on the same SCA workload, timed on the
             host cores of this machine; `dcn` adds the DCN goldens (NCHW: configs[0]
             and res4 / res5 fp32; NHWC: res4 / res5 on fp16-rounded inputs)
Cold-cache protocol (default): a 1 GiB buffer is overwritten before every timed launch so
L2 and the 256 MB MALL hold none of the inputs; --warm times back-to-back launches.
Every timing runs the W warm-up launches, then untimed steps of the timed protocol for
--settle-ms of wall time (default SETTLE_MS), then the K timed steps: after an idle gap of 0.2 s or more (input
set-up, the CPU baseline) the device clocks back up over about 20-30 ms of load, and the
first cold SCA launches measured 394 us against 369 us steady (config.settle_ms).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "bev-kernels_amd")
for _p in (ROOT, PKG):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
SETTLE_MS = 50.0
MFMA_PEAK_TFLOPS = {"fp16": 2516.6, "bf16": 2516.6, "fp32": 157.3}
METRIC = ("MSDA fwd µs + HBM GB/s (BEVFormer SCA); DCNv2 NHWC fwd µs + MFMA TFLOP/s")
COUNTER_FILE = os.path.join(ROOT, "profiles", "msda_sca_fp32_counters.txt")
DCN_COUNTER_FILE = os.path.join(ROOT, "profiles", "dcn_res4_fp16_counters.txt")


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--warm", action="store_true", help="no cache flush between launches")
    ap.add_argument("--settle-ms", type=float, default=SETTLE_MS,
                    help="untimed steps before each timing, in ms of wall time")
    ap.add_argument("--no-configs", action="store_true", help="headline lines only")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", default=None, help="run one configuration (profiling)")
    return ap.parse_args()


def dtype_of(name):
    import torch
    return {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[name]


class Timer:
    """Times launches of `fn` with HIP events on torch's current stream (the stream the
    library enqueues on), optionally after a cache-flushing write."""

    def __init__(self, cold: bool, settle_ms: float = SETTLE_MS):
        import torch
        self.torch = torch
        self.cold = cold
        self.settle_ms = settle_ms
        self.flush_buf = torch.empty(1 << 28, dtype=torch.float32, device="cuda") if cold else None

    def step(self, fn, i):
        if self.cold:
            self.flush_buf.fill_(float(i))
        fn()

    def run(self, fn, steps, warmup):
        torch = self.torch
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize()
        # untimed steps of the timed protocol for settle_ms of wall time
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < self.settle_ms * 1e-3:
            for i in range(4):
                self.step(fn, i)
            torch.cuda.synchronize()
        times = []
        t0 = time.perf_counter()
        for i in range(steps):
            if self.cold:
                self.flush_buf.fill_(float(i))
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record()
            fn()
            e.record()
            times.append((s, e))
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) / steps
        us = [s.elapsed_time(e) * 1e3 for s, e in times]
        return statistics.mean(us), statistics.median(us), wall * 1e6


def msda_case(name, dtype, cache):
    """Device inputs and the kernel call of one MSDA configuration."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    if name not in cache:
        cache[name] = inputs.msda_inputs(name)
    d = cache[name]
    dev = torch.device("cuda")
    v = d["value"].to(dtype).to(dev)
    ss = d["spatial_shapes"].to(dev)
    lsi = d["level_start_index"].to(dev)
    loc = d["sampling_loc"].to(dtype).to(dev)
    att = d["attn_weight"].to(dtype).to(dev)
    es = v.element_size()
    nbytes = (v.numel() + loc.numel() + att.numel() + v.shape[0] * loc.shape[1] * v.shape[2]
              * v.shape[3]) * es
    return (lambda: ext.forward(v, ss, lsi, loc, att, 64, False)), nbytes


def dcn_fused_case(name, dtype, cache, batch=None):
    """Fused NHWC kernel call of one DCN configuration (weight packed once, untimed, as a
    module does on its first call); batch overrides the configuration's image count."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    key = name if batch is None else f"{name}_b{batch}"
    if key not in cache:
        cache[key] = inputs.nchw_to_nhwc(inputs.dcn_inputs(name, batch=batch))
    d = cache[key]
    dev = torch.device("cuda")
    x = d["x"].to(dtype).to(dev)
    off = d["offset"].to(dtype).to(dev)
    msk = d["mask"].to(dtype).to(dev)
    w_packed = ext.dcn_pack_weight(d["weight"].to(dtype).to(dev).contiguous())
    B, H, W, C = x.shape
    Cout = d["weight"].shape[0]
    out = torch.empty(B, H, W, Cout, dtype=dtype, device=dev)
    flops = 2.0 * B * H * W * 9 * C * Cout
    return (lambda: ext.dcn_fused_fwd_nhwc(x, off, msk, w_packed, None, B, C, H, W, H, W, Cout, 3, 3,
                                           1, 1, 1, 1, 1, 1, out)), flops


def dcn_mega_case(name, dtype, cache):
    """One-launch full forward (offset conv + sigmoid + deformable gather + GEMM) of one DCN
    configuration, weights packed once (untimed). Work: 2*M*K*(Cout + 3T) flops (the offset
    conv and the deformable conv)."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    if name not in cache:
        cache[name] = inputs.nchw_to_nhwc(inputs.dcn_inputs(name))
    d = cache[name]
    dev = torch.device("cuda")
    x = d["x"].to(dtype).to(dev)
    B, H, W, C = x.shape
    Cout = d["weight"].shape[0]
    g = torch.Generator().manual_seed(13)
    w_off = (1.5 / (9 * C) ** 0.5 * torch.randn(27, C, 3, 3, generator=g)).to(dtype).to(dev)
    b_off = (0.5 * torch.randn(27, generator=g)).to(dev)
    wo_packed = ext.dcn_pack_weight(w_off.contiguous())
    w_packed = ext.dcn_pack_weight(d["weight"].to(dtype).to(dev).contiguous())
    y = torch.empty(B * H * W, 27, dtype=torch.float32, device=dev)
    out = torch.empty(B, H, W, Cout, dtype=dtype, device=dev)
    flops = 2.0 * B * H * W * 9 * C * (Cout + 27)
    return (lambda: ext.dcn_mega_fwd_nhwc(x, wo_packed, b_off, w_packed, None, B, C, H, W, H, W,
                                          Cout, 3, 3, 1, 1, 1, 1, 1, 1, False, y, out)), flops


def dcn_front_case(name, dtype, cache):
    """Fused front end (offset conv + sigmoid + gather into the column buffer) of one DCN
    configuration. Algorithmic bytes: x read once, columns written once, w_off and b_off."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    if name not in cache:
        cache[name] = inputs.nchw_to_nhwc(inputs.dcn_inputs(name))
    d = cache[name]
    dev = torch.device("cuda")
    x = d["x"].to(dtype).to(dev)
    B, H, W, C = x.shape
    g = torch.Generator().manual_seed(11)
    w_off = (2.0 / (9 * C) ** 0.5 * torch.randn(27, 9, C, generator=g)).to(dtype).to(dev)
    b_off = torch.randn(27, generator=g).to(dev)
    col = torch.empty(B * H * W, 9 * C, dtype=dtype, device=dev)
    es = x.element_size()
    nbytes = x.numel() * es + col.numel() * es + w_off.numel() * es + 27 * 4
    return (lambda: ext.modulated_deformable_fused_im2col_nhwc_cuda(
        x, w_off, b_off, B, C, H, W, H, W, 3, 3, 1, 1, 1, 1, 1, 1, 1, col)), nbytes


def msda_bwd_case(name, dtype, cache):
    """MSDA backward (ext.backward) of one configuration. Algorithmic bytes: value,
    sampling_loc, attn_weight and grad_output read once; grad_value, grad_sampling_loc and
    grad_attn_weight written once (in the input dtype)."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    if name not in cache:
        cache[name] = inputs.msda_inputs(name)
    d = cache[name]
    dev = torch.device("cuda")
    v = d["value"].to(dtype).to(dev)
    ss = d["spatial_shapes"].to(dev)
    lsi = d["level_start_index"].to(dev)
    loc = d["sampling_loc"].to(dtype).to(dev)
    att = d["attn_weight"].to(dtype).to(dev)
    B, S, NH, D = v.shape
    g = torch.Generator().manual_seed(17)
    go = torch.randn(B, loc.shape[1], NH * D, generator=g).to(dtype).to(dev)
    gv = torch.zeros_like(v)
    gl = torch.empty_like(loc)
    ga = torch.empty_like(att)
    es = v.element_size()
    nbytes = (2 * (v.numel() + loc.numel() + att.numel()) + go.numel()) * es
    return (lambda: ext.backward(v, ss, lsi, loc, att, go, gv, gl, ga, 64, False)), nbytes


def dcn_bwd_case(name, dtype, cache):
    """NHWC column-to-image backward (col2im_nhwc: grad_x, grad_offset, grad_mask) of one
    DCN configuration. Algorithmic bytes: column gradient, x, offset and mask read once;
    fp32 grad_x, grad_offset and grad_mask written once."""
    import torch
    import _modulated_deform_conv_ext as ext
    from oracle import inputs
    if name not in cache:
        cache[name] = inputs.nchw_to_nhwc(inputs.dcn_inputs(name))
    d = cache[name]
    dev = torch.device("cuda")
    x = d["x"].to(dtype).to(dev)
    off = d["offset"].to(dtype).to(dev)
    msk = d["mask"].to(dtype).to(dev)
    B, H, W, C = x.shape
    g = torch.Generator().manual_seed(19)
    dcol = torch.randn(B * H * W, 9 * C, generator=g).to(dtype).to(dev)
    gx = torch.zeros(B, H, W, C, dtype=torch.float32, device=dev)
    goff = torch.empty(B, H, W, 18, dtype=torch.float32, device=dev)
    gmask = torch.empty(B, H, W, 9, dtype=torch.float32, device=dev)
    es = x.element_size()
    nbytes = ((dcol.numel() + x.numel() + off.numel() + msk.numel()) * es
              + (gx.numel() + goff.numel() + gmask.numel()) * 4)
    return (lambda: ext.modulated_deformable_col2im_nhwc_cuda(
        dcol, x, off, msk, B, C, H, W, H, W, 3, 3, 1, 1, 1, 1, 1, 1, 1, gx, goff, gmask)), nbytes


def dcn_nchw_case(name, cache):
    """Module-level fp32 NCHW forward (modulated_deform_conv2d)."""
    import torch
    from modulated_deform_conv import modulated_deform_conv2d
    from oracle import inputs
    key = name + "_nchw"
    if key not in cache:
        cache[key] = inputs.dcn_inputs(name)
    d = cache[key]
    dev = torch.device("cuda")
    x, off, msk, w = (d[k].to(dev) for k in ("x", "offset", "mask", "weight"))
    B, C, H, W = x.shape
    flops = 2.0 * B * H * W * 9 * C * w.shape[0]
    return (lambda: modulated_deform_conv2d(x, off, msk, w, None, 1, 1, 1, 1, 1)), flops


def read_counters(path=COUNTER_FILE):
    """HBM-side bytes per launch from a committed rocprofv3 summary: the kernel's
    FETCH_SIZE / WRITE_SIZE per dispatch, each scaled by what the same counter reads for a
    plain copy of known size (None if the summary is absent)."""
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for line in f:
            line = line.strip()
            if "=" in line and not line.startswith("#"):
                k, v = line.split("=", 1)
                try:
                    vals[k.strip()] = float(v.split()[0])
                except ValueError:
                    pass
    try:
        copy_bytes = vals["copy_bytes_each_way"]
        rd_scale = copy_bytes / (vals["copy_FETCH_SIZE_KiB"] * 1024.0)
        wr_scale = copy_bytes / (vals["copy_WRITE_SIZE_KiB"] * 1024.0)
        traffic = (vals["kernel_FETCH_SIZE_KiB"] * 1024.0 * rd_scale
                   + vals["kernel_WRITE_SIZE_KiB"] * 1024.0 * wr_scale)
        return traffic
    except KeyError:
        return None


def cpu_baseline(cache):
    """The CPU oracle (grid_sample form of MSDA) on the full SCA fp32 workload, all host
    threads; 1 warm-up + median of 3."""
    import torch
    from oracle import inputs
    from oracle import msda as om
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    if "msda_sca" not in cache:
        cache["msda_sca"] = inputs.msda_inputs("msda_sca")
    d = cache["msda_sca"]
    nbytes = 4 * (d["value"].numel() + d["sampling_loc"].numel() + d["attn_weight"].numel()
                  + 6 * 10000 * 256)
    om.forward_grid_sample(**d)
    ts = []
    for _ in range(3):
        t0 = time.perf_counter()
        om.forward_grid_sample(**d)
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(nbytes / t / 1e9, 3), "unit": "GB/s", "cores": cores,
            "kind": "port",
            "sample": f"full SCA workload (6x10000x8 queries, fp32) through the oracle's "
                      f"grid_sample form, torch CPU, {cores} threads, median of 3 = "
                      f"{t * 1e3:.0f} ms, {cpu}",
            "dcn": dcn_cpu_baselines(cores)}


def dcn_cpu_baselines(cores):
    """The DCN CPU goldens on the BASELINE workloads, 1 warm-up + median of 3, fp32 on the
    host cores: the NCHW golden (configs[0]; res4 / res5 fp32 NCHW on 2 of the 6 images)
    and the NHWC golden (whole res4 / res5, fp32 on fp16-rounded inputs, the reference for
    the fp16 / bf16 fused runs). GFLOP/s = 2*M*K*Cout of the sample / median time."""
    import torch
    from oracle import dcn as od
    from oracle import inputs
    rows = []
    # (config, layout, images): the NCHW golden of res4 / res5 on a bounded sample of 2
    # of the 6 images (its Python loop over channel x tap dominates); the rest whole
    for name, layout, imgs in (("dcn_c1", "nchw", None), ("dcn_res4", "nchw", 2),
                               ("dcn_res5", "nchw", 2), ("dcn_res4", "nhwc", None),
                               ("dcn_res5", "nhwc", None)):
        d = inputs.dcn_inputs(name, batch=imgs)
        B, C, H, W = d["x"].shape
        cout = d["weight"].shape[0]
        flops = 2.0 * B * H * W * 9 * C * cout
        if layout == "nchw":
            args = (d["x"], d["offset"], d["mask"], d["weight"], d["bias"])
            fn = lambda: od.forward_nchw(*args, (1, 1), (1, 1), (1, 1))  # noqa: E731
        else:
            dn = inputs.nchw_to_nhwc(d)
            r = {k: (v.to(torch.float16).float() if torch.is_tensor(v) else v)
                 for k, v in dn.items()}
            fn = lambda: od.forward_nhwc(r["x"], r["offset"], r["mask"], r["weight"],  # noqa: E731
                                         r["bias"], 1, 1, 1)
        fn()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        t = statistics.median(ts)
        rows.append({"config": f"{name}_{layout}_golden", "ms": round(t * 1e3, 1),
                     "GFLOP/s": round(flops / t / 1e9, 1), "cores": cores,
                     "sample": (f"{B} of the 6 images" if imgs else f"whole workload (B={B})")
                               + ", fp32, median of 3"})
    return rows


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the operators shard over cameras / batch with no communication: each GPU runs "
              "its own share of the batch; only the one-GPU rate is measured here)",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import _bevk
    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    _bevk.lib()
    torch.backends.cuda.matmul.allow_tf32 = False
    timer = Timer(cold=not args.warm, settle_ms=args.settle_ms)
    cache = {}
    steps, warmup = args.steps, args.warmup

    if args.only:
        kind, _, rest = args.only.partition(":")
        name, _, dt = rest.partition(":")
        if kind == "msda":
            fn, _ = msda_case(name, dtype_of(dt), cache)
        elif kind == "dcn":
            dt, _, b = dt.partition(":")
            fn, _ = dcn_fused_case(name, dtype_of(dt), cache, batch=int(b) if b else None)
        elif kind == "dcn_nchw":
            fn, _ = dcn_nchw_case(name, cache)
        elif kind == "dcn_mega":
            fn, _ = dcn_mega_case(name, dtype_of(dt), cache)
        elif kind == "dcn_front":
            fn, _ = dcn_front_case(name, dtype_of(dt), cache)
        elif kind == "msda_bwd":
            fn, _ = msda_bwd_case(name, dtype_of(dt), cache)
        elif kind == "dcn_bwd":
            fn, _ = dcn_bwd_case(name, dtype_of(dt), cache)
        elif kind == "copy":
            # plain copy of known size: the counter calibration reference
            n = int(name) if name else 256 << 20
            src = torch.empty(n // 4, dtype=torch.float32, device="cuda").fill_(1.0)
            dst = torch.empty_like(src)
            fn = lambda: dst.copy_(src)  # noqa: E731
        else:
            raise SystemExit(f"unknown --only {args.only}")
        mean_us, med_us, wall_us = timer.run(fn, steps, warmup)
        print(json.dumps({"only": args.only, "mean_us": round(mean_us, 2),
                          "median_us": round(med_us, 2)}), flush=True)
        return

    # ---- headline: MSDA SCA fp32 -------------------------------------------------------
    fn, nbytes = msda_case("msda_sca", torch.float32, cache)
    mean_us, med_us, wall_us = timer.run(fn, steps, warmup)
    gbs = nbytes / (mean_us * 1e-6) / 1e9
    traffic = read_counters()
    dcn_traffic = read_counters(DCN_COUNTER_FILE)
    warm_us = Timer(cold=False, settle_ms=args.settle_ms).run(fn, steps, warmup)[0]

    # ---- secondary: DCN res4 fp16 fused, on the configs protocol (>= 100 launches) ------
    reps, wu = max(100, steps), max(10, warmup)   # per row: >= 100 timed after >= 10
    dfn, flops = dcn_fused_case("dcn_res4", torch.float16, cache)
    d_mean, d_med, _ = timer.run(dfn, reps, wu)
    tflops = flops / (d_mean * 1e-6) / 1e12

    line = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(mean_us / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded BASELINE distributions)",
        "config": {"workload": "MSDA forward, BEVFormer spatial cross-attention (BASELINE "
                               "configs[4]): B=6 cameras, 4 levels (116x200, 58x100, 29x50, "
                               "15x25), Len_in=30825, Len_q=10000, 8 heads x 32, 8 points",
                   "cache": "warm" if args.warm else "cold (1 GiB overwrite before each launch)",
                   "median_us": round(med_us, 2), "warm_mean_us": round(warm_us, 2),
                   "settle_ms": args.settle_ms,
                   "algorithmic_bytes": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": None if traffic is None else round(traffic)},
        "secondary": {
            "metric": "DCNv2 NHWC fused forward, res4 (B=6, 256->256, 58x100), fp16",
            "us": round(d_mean, 2), "median_us": round(d_med, 2), "launches": reps,
            "value": round(tflops, 2), "unit": "TFLOP/s",
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2),
                         "peak": MFMA_PEAK_TFLOPS["fp16"], "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_PEAK_TFLOPS["fp16"], 4),
                         "traffic": None if dcn_traffic is None else round(dcn_traffic)}},
    }

    if not args.no_configs:
        rows = []
        for name in ("msda_sca", "msda_tsa", "msda_detr"):
            for dt in ("fp32", "fp16", "bf16"):
                f, nb = msda_case(name, dtype_of(dt), cache)
                m, _, _ = timer.run(f, reps, wu)
                g = nb / (m * 1e-6) / 1e9
                rows.append({"config": name, "dtype": dt, "us": round(m, 2),
                             "GB/s": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4)})
        for name in ("dcn_res4", "dcn_res5"):
            for dt in ("fp16", "bf16", "fp32"):
                f, fl = dcn_fused_case(name, dtype_of(dt), cache)
                if name == "dcn_res4" and dt == "fp16":
                    m = d_mean  # the secondary's launches: one figure for this kernel
                else:
                    m, _, _ = timer.run(f, reps, wu)
                tf = fl / (m * 1e-6) / 1e12
                rows.append({"config": name + "_nhwc_fused", "dtype": dt, "us": round(m, 2),
                             "TFLOP/s": round(tf, 2),
                             "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4)})
            f, fl = dcn_nchw_case(name, cache)
            m, _, _ = timer.run(f, reps, wu)
            tf = fl / (m * 1e-6) / 1e12
            rows.append({"config": name + "_nchw_module", "dtype": "fp32", "us": round(m, 2),
                         "TFLOP/s": round(tf, 2),
                         "frac_mfma": round(tf / MFMA_PEAK_TFLOPS["fp32"], 4)})
            for dt in ("fp16", "bf16"):
                f, fl = dcn_mega_case(name, dtype_of(dt), cache)
                m, _, _ = timer.run(f, reps, wu)
                tf = fl / (m * 1e-6) / 1e12
                rows.append({"config": name + "_mega_one_launch", "dtype": dt,
                             "us": round(m, 2), "TFLOP/s": round(tf, 2),
                             "frac_mfma": round(tf / MFMA_PEAK_TFLOPS[dt], 4)})
            # the same layer at other batch sizes (the persistent schedule at any row count)
            for b in ((1, 4) if name == "dcn_res4" else (1,)):
                f, fl = dcn_fused_case(name, torch.float16, cache, batch=b)
                m, _, _ = timer.run(f, reps, wu)
                tf = fl / (m * 1e-6) / 1e12
                rows.append({"config": f"{name}_nhwc_fused_b{b}", "dtype": "fp16",
                             "us": round(m, 2), "TFLOP/s": round(tf, 2),
                             "frac_mfma": round(tf / MFMA_PEAK_TFLOPS["fp16"], 4)})
            f, nb = dcn_front_case(name, dtype_of("fp16"), cache)
            m, _, _ = timer.run(f, reps, wu)
            g = nb / (m * 1e-6) / 1e9
            rows.append({"config": name + "_front_end", "dtype": "fp16", "us": round(m, 2),
                         "GB/s": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4)})
            for dt in ("fp16", "fp32"):
                f, nb = dcn_bwd_case(name, dtype_of(dt), cache)
                m, _, _ = timer.run(f, reps, wu)
                g = nb / (m * 1e-6) / 1e9
                rows.append({"config": name + "_col2im_nhwc_backward", "dtype": dt,
                             "us": round(m, 2), "GB/s": round(g, 1),
                             "frac_hbm": round(g / HBM_PEAK_GBS, 4)})
        for name in ("msda_sca", "msda_tsa", "msda_detr"):
            for dt in ("fp32", "fp16", "bf16"):
                f, nb = msda_bwd_case(name, dtype_of(dt), cache)
                m, _, _ = timer.run(f, reps, wu)
                g = nb / (m * 1e-6) / 1e9
                rows.append({"config": name + "_backward", "dtype": dt, "us": round(m, 2),
                             "GB/s": round(g, 1), "frac_hbm": round(g / HBM_PEAK_GBS, 4)})
        line["configs"] = rows

    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cache)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
