#!/usr/bin/env python3
"""End-to-end SCUNet-color throughput on one MI355X, with per-kernel roofline figures and
the reference CPU path (the oracle restatement of src/cpu.rs) timed beside it.

A step is one whole-image forward of SCUNet colour (in_nc 3, dim 64, config [4]*7,
window 8, head_dim 32, seeded random-init fp32 weights) on benchmark config 3: a
1x3x1080x1920 seeded noisy image already resident in HBM, replicate-padded to
1088x1920 and cropped back on the device (scunet_hip_run_device: the backend::run
contract with pad and crop fused into the first and last convolution).

value = 1920*1080 input pixels / mean step time, in Mpx/s (the reference counts input
pixels, examples/bench.rs:191). Per-kernel device times come from HIP event pairs that
the library records around every launch on its own stream during the timed steps; the
fp16-operand mode is timed after them and reported in its own sub-object (fp16_mode), as is
the all-fp32-MFMA mode (fp32_mfma_mode). The default fp32 mode forms most products from an
exact three-way bf16 split of the fp32 operands on the bf16 matrix cores (SPLIT_CLASSES).

Usage: python bench.py [--gpus 1] [--steps 10] [--warmup 5] [--no-cpu-baseline] [--no-fp16]
                       [--no-fp32-mfma]
"""
import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "scunet-rs_amd"))

METRIC = "megapixels/sec end-to-end SCUNet-color 1920x1088; attention kernel TFLOP/s"
PEAK_FP32_TFLOPS = 157.3      # MI355X dense fp32 matrix
PEAK_FP16_TFLOPS = 2500.0     # MI355X dense fp16 matrix (the fp16-operand mode's products)
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 matrix (the split-operand fp32 products)
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
# The 3x3 convolutions run as Winograd F(2x2,3x3) unless SCUNET_HIP_DIRECT3X3 is set (or in
# the fp16 mode, which uses a direct kernel): the library counts the direct convolution's
# 18*cin*cout FLOP per pixel for every path, the Winograd kernel executes 16 products of
# (cout x cin) per 2x2 output tile, i.e. 8*cin*cout FLOP per pixel, on the MFMA units.
WINOGRAD_EXECUTED = 8.0 / 18.0
# The default fp32 mode forms these classes' products from an exact three-way bf16 split of
# both fp32 operands: six bf16 part products per fp32 multiply-add on the bf16 matrix cores
# (fp32 accumulation). Their executed work is 6x the algorithmic FLOP, against the bf16 peak.
# conv3x3_split is the Winograd 3x3 at cin = cout = 32 (level 0) in that form: 6 x 8/18; the
# tail forms its products from split operands too.
SPLIT_CLASSES = {"conv1x1", "conv1x1_chain", "mlp_fused", "msa_fused", "tblock_fused", "up2x2", "down2x2",
                 "conv3x3_split", "tail"}
SPLIT_EXECUTED = 6.0
PRODUCTS = ("fp32 operands, planes and accumulation; the products of the split classes (" +
            ", ".join(sorted(SPLIT_CLASSES)) + ") on the bf16 matrix cores from an exact three-way bf16 split "
            "of each operand (six part products, dropped terms < 2^-25 |ab|), the rest on the fp32 matrix cores")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def roofline_of(name, launches, ms, flop, byts, peak_tflops=PEAK_FP32_TFLOPS, executed=1.0):
    """Roofline figures of one kernel class. flop/byts are the library's algorithmic counts
    summed over the launches; `executed` scales flop to what the MFMA units execute (the
    Winograd 3x3), so `achieved` and `frac` are executed rates and frac <= 1 by
    construction. The bound is the side of the ridge the executed work falls on."""
    xflop = flop * executed
    ridge = peak_tflops * 1e12 / (PEAK_HBM_GBS * 1e9)
    base = {"kernel": name, "traffic": None, "launches": launches, "avg_launch_ms": round(ms / launches, 5),
            "algorithmic_flop_per_launch": xflop / launches, "algorithmic_bytes_per_launch": byts / launches}
    if xflop / max(byts, 1.0) >= ridge:
        ach = xflop / (ms * 1e-3) / 1e12
        return dict(base, bound="mfma", achieved=round(ach, 3), peak=peak_tflops, unit="TFLOP/s",
                    frac=round(ach / peak_tflops, 4))
    ach = byts / (ms * 1e-3) / 1e9
    return dict(base, bound="hbm", achieved=round(ach, 1), peak=PEAK_HBM_GBS, unit="GB/s",
                frac=round(ach / PEAK_HBM_GBS, 4))


def class_table(rows, steps, peak_tflops, winograd, split=frozenset()):
    """Per kernel class (rows are per class and UNet level "@Lk"): roofline figures, share of
    device time and the per-level breakdown, sorted by device time. Classes in `split` run
    split-operand products: executed FLOP 6x the algorithmic, against the bf16 peak."""
    total_ms = max(sum(r[2] for r in rows), 1e-9)
    classes = {}
    for name, n, ms, flop, byts in rows:
        agg = classes.setdefault(name.split("@")[0], [0, 0.0, 0.0, 0.0])
        agg[0] += n
        agg[1] += ms
        agg[2] += flop
        agg[3] += byts
    out = []
    for base, (n, ms, flop, byts) in sorted(classes.items(), key=lambda kv: -kv[1][1]):
        wino = (winograd and base == "conv3x3") or base == "conv3x3_split"
        ex = WINOGRAD_EXECUTED if wino else 1.0
        pk = peak_tflops
        if base in split:
            ex, pk = ex * SPLIT_EXECUTED, PEAK_BF16_TFLOPS
        k = roofline_of(base, n, ms, flop, byts, pk, ex)
        k["share"] = round(ms / total_ms, 4)
        if base in split:
            k["products"] = "split bf16 x6: achieved/frac count the six bf16 part products per fp32 multiply-add"
            k["fp32_equiv_tflops"] = round(flop / (ms * 1e-3) / 1e12, 3)
        if wino:
            k["algorithm"] = ("winograd F(2x2,3x3): achieved/frac count the 8*cin*cout FLOP per pixel the MFMA "
                              "units execute; direct_equiv_tflops counts the direct convolution's 18*cin*cout")
            k["direct_equiv_tflops"] = round(flop / (ms * 1e-3) / 1e12, 3)
        k["levels"] = {}
        for name, n2, ms2, flop2, byts2 in rows:
            if name.split("@")[0] == base and "@" in name:
                lv = roofline_of(name, n2, ms2, flop2, byts2, pk, ex)
                k["levels"][name.split("@")[1]] = {"achieved": lv["achieved"], "unit": lv["unit"],
                                                   "frac": lv["frac"], "avg_launch_ms": lv["avg_launch_ms"],
                                                   "ms_per_step": round(ms2 / steps, 4)}
        out.append(k)
    return out


def measured_traffic():
    """HBM bytes per launch per kernel class, from the calibrated FETCH_SIZE/WRITE_SIZE
    counter passes summarised in profiles/counters_1080p.md (machine-readable copy:
    profiles/traffic_1080p.json). None when the file is absent."""
    p = os.path.join(REPO, "profiles", "traffic_1080p.json")
    if not os.path.exists(p):
        return {}
    with open(p) as f:
        return json.load(f).get("classes", {})


def cpu_baseline(weights_path, x, rows, iters):
    """The oracle (C++ restatement of the reference's src/cpu.rs, OpenMP over all host
    threads; it stands in for the reference's Rust CPU backend, which cannot be built here)
    on a bounded sample of the benchmark's own input: the top `rows` rows of the 1080p
    image, forwarded as one whole image (the same per-pixel work), 1 untimed warmup then
    `iters` timed runs (the protocol of the reference's examples/bench.rs:151-214 for
    configs 1-3). value = the median run's Mpx/s."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle
    wt = oracle.Weights.load(weights_path)
    sample = np.ascontiguousarray(x[:, :rows, :])
    c, h, w = sample.shape
    oracle.run(wt, sample)
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        oracle.run(wt, sample)
        ts.append(time.perf_counter() - t0)
    ts.sort()
    med = ts[len(ts) // 2]
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {"value": round(h * w / med / 1e6, 5), "unit": "Mpx/s", "cores": oracle.threads(), "kind": "port",
            "sample": f"a strip, not the full frame: the top {h} of the benchmark image's 1080 rows "
                      f"({c}x{h}x{w}, {h * w / 1e6:.3f} Mpx) forwarded as one image through "
                      f"oracle/scunet_oracle.cpp (the C++ restatement of src/cpu.rs) on {oracle.threads()} OpenMP "
                      f"threads; 1 warmup + {iters} timed runs, value from the median",
            "iterations": iters, "warmup": 1,
            "seconds": [round(t, 3) for t in ts], "median_s": round(med, 3),
            "spread_pct": round(100.0 * (ts[-1] - ts[0]) / med, 2),
            "mpx_s_min_max": [round(h * w / ts[-1] / 1e6, 5), round(h * w / ts[0] / 1e6, 5)],
            "omp_threads": oracle.threads(), "nproc": os.cpu_count(), "affinity_cpus": affinity,
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}


def attention_sweep(be, wpath, iters):
    """benchmark config 5: the isolated window-attention core (the reference's kernel boundary,
    qkv -> out, cuda.rs:767-808) at each level's 1920x1088 window grid, W and SW. x ~ N(0,1)
    [nw*64][C]; qkv = x Wqkv^T + b with the level's seeded embedding weights; rel-pos
    tables ~ N(0, 0.02) in upstream's [225][heads] storage, re-viewed to [heads][15][15]."""
    import numpy as np
    from scunet_hip.safetensors_io import read_safetensors
    t, _ = read_safetensors(wpath)
    out = []
    for level in range(4):
        c = 32 << level
        heads = c // 32
        nwh, nww = 136 >> level, 240 >> level
        nw = nwh * nww
        rng = np.random.default_rng(500 + level)
        x = rng.standard_normal((nw * 64, c), dtype=np.float32)
        name = ["m_down1.0", "m_down2.0", "m_down3.0", "m_body.0"][level] + ".trans_block.msa.embedding_layer"
        qkv = np.ascontiguousarray(x @ np.asarray(t[name + ".weight"]).T + np.asarray(t[name + ".bias"]),
                                   dtype=np.float32)
        del x
        raw = np.clip(rng.standard_normal((225, heads)) * 0.02, -0.04, 0.04)
        rp = raw.reshape(15, 15, heads).transpose(0, 2, 1).transpose(1, 0, 2).astype(np.float32)
        qp = be.malloc(qkv.nbytes)
        op = be.malloc(qkv.nbytes // 3)
        be.h2d(qp, qkv)
        for shift in (0, 4):
            ms = be.bench_attn(qp, rp, op, nwh, nww, c, heads, shift, iters)
            flop = 16384.0 * c * nw
            byts = 4.0 * 64 * nw * 4 * c
            out.append({"level": level, "C": c, "heads": heads, "windows": nw, "shift": shift,
                        "ms": round(ms, 5), "tflops": round(flop / (ms * 1e-3) / 1e12, 3),
                        "gbs": round(byts / (ms * 1e-3) / 1e9, 1),
                        "frac_hbm": round(byts / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)})
            log(f"  attention C={c:3d} nw={nw:5d} shift={shift}: {ms * 1e3:8.1f} us, "
                f"{out[-1]['tflops']:7.2f} TFLOP/s, {out[-1]['gbs']:7.1f} GB/s ({100 * out[-1]['frac_hbm']:.1f}% of HBM)")
        be.free(qp)
        be.free(op)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-rows", type=int, default=192,
                    help="rows of the 1080p input the CPU baseline forwards (a multiple of 64)")
    ap.add_argument("--cpu-iters", type=int, default=3, help="timed CPU-baseline runs (after 1 warmup)")
    ap.add_argument("--no-kernel-events", action="store_true",
                    help="time the steps without the per-launch event pairs")
    ap.add_argument("--no-attn-sweep", action="store_true", help="skip the config-5 attention sweep")
    ap.add_argument("--no-fp16", action="store_true", help="skip the fp16-operand mode's line")
    ap.add_argument("--no-fp32-mfma", action="store_true", help="skip the all-fp32-MFMA mode's line")
    ap.add_argument("--profile-fp16", action="store_true", help="with --profile-pass: the forward in the fp16 mode")
    ap.add_argument("--profile-pass", action="store_true",
                    help="for rocprofv3 counter runs: one forward plus one 256 MiB device copy (the "
                         "calibration kernel), nothing else; prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        log("bench.py: this build runs one image on one GPU; multi-GPU runs are not part of it "
            "(one image per GPU shards with no communication; one image over several GPUs would "
            "split into 64-row bands with halo exchange). Use --gpus 1.")
        sys.exit(2)

    import numpy as np
    import scunet_hip
    from scunet_hip import synth

    wpath = synth.weights_file(seed=0)
    x = synth.config_input(3)                     # [3][1080][1920]
    c, h, w = x.shape
    plan = scunet_hip.Plan(h, w)
    be = scunet_hip.Hip(wpath)
    xp = be.malloc(x.nbytes)
    yp = be.malloc(x.nbytes)
    be.h2d(xp, x)
    log(f"bench: SCUNet-color {c}x{h}x{w} (padded {plan.hp}x{plan.wp}) on {be.name()}, "
        f"warmup {args.warmup}, steps {args.steps}")

    if args.profile_pass:
        if args.profile_fp16:
            be.set_precision("fp16")
            be.run_device(xp, c, h, w, yp)      # the fp16 weight copies are built before the pass
            be.synchronize()
        nbytes = 256 << 20
        a_, b_ = be.malloc(nbytes), be.malloc(nbytes)
        be.copy(b_, a_, nbytes)
        be.synchronize()
        be.run_device(xp, c, h, w, yp)
        be.synchronize()
        be.free(a_)
        be.free(b_)
        log("bench: profile pass done (1 forward, 1 copy of 256 MiB)")
        be.close()
        return

    for _ in range(args.warmup):
        be.run_device(xp, c, h, w, yp)
    be.synchronize()
    be.profile(not args.no_kernel_events)
    be.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        be.run_device(xp, c, h, w, yp)
    be.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    rows = be.profile_rows() if not args.no_kernel_events else []
    be.profile(False)
    y = be.d2h(np.empty_like(x), yp)
    if not np.isfinite(y).all():
        raise RuntimeError("non-finite output")
    mpx = h * w / dt / 1e6
    log(f"bench: {dt * 1e3:.2f} ms/step, {mpx:.2f} Mpx/s")

    # Per-step distribution: the same steps again, each synchronised on its own and without
    # the per-launch events (min and median, as the reference's bench reports them).
    per = []
    for _ in range(args.steps):
        t1 = time.perf_counter()
        be.run_device(xp, c, h, w, yp)
        be.synchronize()
        per.append(time.perf_counter() - t1)
    per.sort()
    step_min, step_med = per[0], per[len(per) // 2]
    log(f"bench: per-step (synchronised, no events) min {step_min * 1e3:.2f} ms, median {step_med * 1e3:.2f} ms")
    # Host to host: backend::run on host buffers (H2D, pad, forward, crop, D2H). Reported
    # beside the device-resident figure, never as it.
    be.run_fused(x)
    h2h = []
    for _ in range(3):
        t1 = time.perf_counter()
        be.run_fused(x)
        h2h.append(time.perf_counter() - t1)
    h2h_med = sorted(h2h)[1]
    log(f"bench: host to host (scunet_hip_run, PCIe included) {h2h_med * 1e3:.2f} ms, {h * w / h2h_med / 1e6:.2f} Mpx/s")
    fp = be.footprint()

    # The all-fp32-MFMA mode (SCUNET_HIP_FP32_MFMA: every product on the fp32 matrix cores),
    # timed the same way and reported beside the default, with its difference from it.
    mfma_mode = None
    if not args.no_fp32_mfma:
        be.set_precision("fp32_mfma")
        for _ in range(args.warmup):
            be.run_device(xp, c, h, w, yp)
        be.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            be.run_device(xp, c, h, w, yp)
        be.synchronize()
        dtm = (time.perf_counter() - t1) / args.steps
        ym = be.d2h(np.empty_like(x), yp)
        be.set_precision("fp32")
        mfma_mode = {"value": round(h * w / dtm / 1e6, 3), "unit": "Mpx/s", "ms_per_step": round(dtm * 1e3, 3),
                     "max_abs_vs_default": float(np.abs(ym.astype(np.float64) - y.astype(np.float64)).max()),
                     "note": "scunet_hip_set_precision(SCUNET_HIP_FP32_MFMA): every product on the fp32 matrix "
                             "cores (v_mfma_f32_16x16x4_f32); same planes and accumulation as the default"}
        log(f"bench: fp32-MFMA mode {dtm * 1e3:.2f} ms/step, {mfma_mode['value']:.2f} Mpx/s, max |diff| vs default "
            f"{mfma_mode['max_abs_vs_default']:.2e}")

    # The fp16-operand mode (fp16 MFMA operands, fp32 accumulation and planes), reported
    # beside the fp32 headline with its error against the fp32 output of the same input.
    fp16 = None
    if not args.no_fp16:
        be.set_precision("fp16")
        for _ in range(args.warmup):
            be.run_device(xp, c, h, w, yp)
        be.synchronize()
        be.profile(not args.no_kernel_events)
        be.synchronize()
        t1 = time.perf_counter()
        for _ in range(args.steps):
            be.run_device(xp, c, h, w, yp)
        be.synchronize()
        dt16 = (time.perf_counter() - t1) / args.steps
        rows16 = be.profile_rows() if not args.no_kernel_events else []
        be.profile(False)
        y16 = be.d2h(np.empty_like(x), yp)
        be.set_precision("fp32")
        d = y16.astype(np.float64) - y.astype(np.float64)
        mse = float(np.mean(d * d))
        fp16 = {"value": round(h * w / dt16 / 1e6, 3), "unit": "Mpx/s", "ms_per_step": round(dt16 * 1e3, 3),
                "max_abs_vs_fp32": float(np.abs(d).max()),
                "psnr_db_vs_fp32": round(10 * np.log10(1.0 / mse), 2) if mse > 0 else None,
                "tolerance": {"max_abs": 4e-3, "psnr_db": 70.0},
                "note": "scunet_hip_set_precision(SCUNET_HIP_FP16): fp16 MFMA operands, fp32 accumulation, "
                        "fp32 planes/LayerNorm/softmax/GELU; not the headline (the reference path is fp32)"}
        if rows16:
            k16 = class_table(rows16, args.steps, PEAK_FP16_TFLOPS, winograd=False)
            flop16 = sum(r[3] for r in rows16) / args.steps
            byts16 = sum(r[4] for r in rows16) / args.steps
            dev16 = sum(r[2] for r in rows16) / args.steps
            fp16["forward"] = {"tflops": round(flop16 / (dev16 * 1e-3) / 1e12, 2),
                               "frac_of_fp16_peak": round(flop16 / (dev16 * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                               "algorithmic_gbs": round(byts16 / (dev16 * 1e-3) / 1e9, 1),
                               "frac_of_hbm": round(byts16 / (dev16 * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                               "device_ms_per_step": round(dev16, 3),
                               "note": "whole forward: algorithmic FLOP (all products direct in this mode) and "
                                       "bytes over the summed per-launch device times, against the 2.5 PFLOP/s "
                                       "dense fp16 MFMA peak and 8 TB/s"}
            fp16["roofline"] = k16[0]
            fp16["kernels"] = k16
        log(f"bench: fp16 mode {dt16 * 1e3:.2f} ms/step, {fp16['value']:.2f} Mpx/s, max |diff| vs fp32 "
            f"{fp16['max_abs_vs_fp32']:.2e}, PSNR {fp16['psnr_db_vs_fp32']} dB")
        if "forward" in fp16:
            f = fp16["forward"]
            log(f"bench: fp16 mode forward {f['tflops']} TFLOP/s ({100 * f['frac_of_fp16_peak']:.1f}% of the fp16 "
                f"peak), {f['algorithmic_gbs']} GB/s ({100 * f['frac_of_hbm']:.1f}% of HBM)")

    kernels = class_table(rows, args.steps, PEAK_FP32_TFLOPS, winograd=not os.environ.get("SCUNET_HIP_DIRECT3X3"),
                          split=SPLIT_CLASSES)
    for k in kernels:
        log(f"  {k['kernel']:>14}: {k['launches']:5d} launches, {k['avg_launch_ms'] * 1e3:9.1f} us avg, "
            f"{k['achieved']:9.2f} {k['unit']} ({100 * k['frac']:.1f}% of {k['bound']}), share {100 * k['share']:.1f}%")
        for lvl, v in sorted(k["levels"].items()):
            log(f"  {'':>14}   {lvl}: {v['avg_launch_ms'] * 1e3:9.1f} us avg, {v['ms_per_step']:7.3f} ms/step, "
                f"{v['achieved']:9.2f} {v['unit']} ({100 * v['frac']:.1f}%)")
    # Hardware-counter figures per class (profiles/counters_1080p.md): HBM bytes per launch
    # and the MFMA-busy fraction, beside the event-timed rates above.
    traffic = measured_traffic()
    for k in kernels:
        t = traffic.get(k["kernel"])
        if t and t["launches"] * args.steps == k["launches"]:
            k["traffic"] = round(t["traffic_bytes_per_launch"])
            k["traffic_source"] = "profiles/counters_1080p.md"
            if "mfma_busy_pct" in t:
                k["mfma_busy_counter"] = round(t["mfma_busy_pct"] / 100.0, 4)
    dominant = kernels[0] if kernels else None
    # The forward's window attention runs inside the fused window kernels: msa_fused (LN1,
    # qkv, attention, proj, residual; levels 1-3) and tblock_fused (the same plus the MLP;
    # level 0). The isolated attention core (k_attention) is measured by the config-5 sweep.
    attn = next((k for k in kernels if k["kernel"] == "msa_fused"), None)
    tblock = next((k for k in kernels if k["kernel"] == "tblock_fused"), None)
    attn_tflops = attn["achieved"] if attn else None

    sweep = None
    if not args.no_attn_sweep:
        log("bench: config-5 attention operator sweep")
        sweep = attention_sweep(be, wpath, 20)

    cpu = None
    if not args.no_cpu_baseline:
        log(f"bench: CPU baseline (oracle) on the top {args.cpu_rows} rows of the input, 1 warmup + "
            f"{args.cpu_iters} timed ...")
        cpu = cpu_baseline(wpath, x, args.cpu_rows, args.cpu_iters)
        log(f"bench: CPU baseline {cpu['value']} Mpx/s (median) on {cpu['cores']} threads, runs {cpu['seconds']} s, "
            f"spread {cpu['spread_pct']}%")

    line = {
        "metric": METRIC,
        "value": round(mpx, 3),
        "unit": "Mpx/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded noisy 1080x1920 texture, sigma 15/255; seeded random-init weights)",
        "config": {"workload": "SCUNet-color whole-image forward, 1x3x1080x1920 replicate-padded to 1088x1920 "
                               "(benchmark config 3), device-resident input, pad+crop on device",
                   "in_nc": 3, "dim": 64, "blocks": [4] * 7, "window": 8, "head_dim": 32,
                   "products": PRODUCTS,
                   "kernel_events": not args.no_kernel_events},
        "roofline": dominant,
        "attention_tflops": attn_tflops,
        "attention_roofline": attn,
        "window_transformer_roofline": tblock,
        "attention_sweep": sweep,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "step_ms": {"min": round(step_min * 1e3, 3), "median": round(step_med * 1e3, 3),
                    "note": "per-step synchronised pass without per-launch events"},
        "host_to_host": {"ms": round(h2h_med * 1e3, 3), "mpx_s": round(h * w / h2h_med / 1e6, 3),
                         "note": "scunet_hip_run on host buffers: H2D + pad + forward + crop + D2H, median of 3"},
        "device_bytes": {"weights": fp[0], "scratch": fp[1]},
        "fp16_mode": fp16,
        "fp32_mfma_mode": mfma_mode,
    }
    be.free(xp)
    be.free(yp)
    be.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
