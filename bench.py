#!/usr/bin/env python3
"""TAGI step throughput on one MI355X: forward moments + innovation + backward deltas +
capped update, ResNet-18 at batch 128 on 3x32x32 synthetic inputs (fp32).

    python bench.py [--steps K] [--warmup W] [--workload resnet18|cnn|mlp|transformer]

Prints one JSON line. ``value`` is samples/s over the K timed steps (inputs already in
HBM). The engine's HIP-event timer (events recorded on the launch stream around each
kernel-family entry point) runs in two modes: over the warm-up steps it brackets every
family (the per-family breakdown, and the choice of the dominant MFMA family: the one with
the most algorithmic work); over the timed steps it brackets only that family, whose
algorithmic FLOPs divided by
its measured time give ``roofline.achieved`` (timing every family would add ~500 event
records per step to the timed region). ``cpu_baseline`` times the float32 CPU oracle
(the reference's moment equations in torch CPU ops) on a bounded sample of the same
workload, on the host's cores.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "triton-tagi_amd"))
sys.path.insert(0, str(ROOT))

METRIC = "TAGI step samples/sec (fwd+bwd+update) ResNet-18 b128 fp32; % MFMA/HBM peak"
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
TIMER_STEPS = 5  # timed steps (the last ones) that carry the live per-launch timer
MFMA_FAMILIES = ("conv_fwd", "conv_bwd_delta", "conv_wgrad", "linear_fwd", "linear_bwd_delta", "linear_wgrad",
                 "bmm_fwd", "bmm_shared", "attn_scores")
WORKLOAD_DESC = {
    "resnet18": "TAGI ResNet-18 (BasicBlock 64/128/256/512, BatchNorm2D, Add, AvgPool4, Linear 512-10, Remax), "
                "batch 128, 3x32x32 ~ N(0,1), gain 0.1, sigma_v 0.05, full fwd+bwd+update step",
    "cnn": "TAGI CNN (3x Conv5x5 pad2/ReLU/AvgPool2, Linear 1024-256-10, Remax), batch 128, 3x32x32",
    "mlp": "TAGI MLP 784-256-128-10 ReLU + Remax, batch 256",
    "transformer": "TAGI transformer block (Embedding 64x256 + PE + MHA-V2 8 heads + RMSNorm + Linear 256-64), "
                   "batch 64, seq 256",
    "mlp_hrc": "TAGI MLP 784-128-11 with a hierarchical-softmax head (10 classes), step_hrc, batch 512",
    "resnet18_hrc": "TAGI ResNet-18 (as resnet18) with the head Linear 512-11 and a hierarchical-softmax "
                    "output (10 classes), step_hrc, batch 128",
    "heads": "bandwidth of the HRC, heteroscedastic, EvenSoftplus, MaxPool2D and LayerNorm kernels at "
             "HBM-bound sizes (one case per kernel, listed in cases)",
    "linear": "TAGI Linear layer microbench, (batch, in, out) = (4096,4096,4096), (8192,1024,4096), "
              "(256,4096,11008): forward moments + backward deltas + capped update",
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(workload: str, batch: int, timed_steps: int = 3):
    """Float32 CPU oracle on the same workload as the GPU run (same architecture, batch,
    seeded priors and inputs), on all the host cores this process may run on: 1 warm-up
    step, then the median of ``timed_steps`` steps; samples/s from the median."""
    import torch

    from oracle import tagi_oracle as O
    from triton_tagi_amd import workloads

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(max(cores, 1))
    w = workloads.build(workload, device="cpu", batch=batch)
    onet = O.mirror_net(w.net, dtype=torch.float32)
    x = w.x.float()
    if w.hrc is not None:
        n_classes = w.hrc.obs.shape[0]

        def step():
            onet.step_hrc(x, w.y, n_classes, w.sigma_v)
    else:
        y = w.y.float()

        def step():
            onet.step(x, y, w.sigma_v)

    step()  # warm-up
    times = []
    for _ in range(timed_steps):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
        log(f"[bench] cpu step {len(times)}: {times[-1]:.2f} s")
    med = statistics.median(times)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {
        "value": w.batch / med,
        "unit": "samples/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": f"{workload} step at batch {w.batch} (the GPU run's workload: same architecture, priors and "
                  f"inputs), fp32 torch CPU ops on {cores} threads (sched_getaffinity), 1 warm-up + median of "
                  f"{timed_steps} steps ({med:.2f} s/step); cpu: {cpu_model}",
    }


def measure_ceilings(dev: str) -> dict:
    """Measured ceilings of this GPU: the fp32 MFMA issue loop at 1, 2 and 4 waves per
    SIMD (the engine's probe kernel), the same loop with 1-8 VALU or LDS instructions per
    MFMA, a 1 GiB device-to-device copy (the HIP runtime's copy
    kernel) and an fp32 GEMM through torch.matmul (hipBLASLt) for comparison."""
    import torch

    from triton_tagi_amd import _lib

    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    st = torch.cuda.current_stream().cuda_stream
    out = {"gpu": props.name, "cus": cus}
    buf = torch.empty(cus * 4 * 256, device=dev)

    def timed(fn, reps):
        fn()
        torch.cuda.synchronize()
        t_end = time.perf_counter() + 0.5  # clock warm-up
        while time.perf_counter() < t_end:
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / 1e3 / reps

    iters = 4000
    for w in (1, 2, 4):
        blocks = cus * w
        s = timed(lambda: _lib.call("tagi_probe_mfma_loop", buf.data_ptr(), blocks, iters, st), 20)
        flops = blocks * 4 * iters * 4 * (32 * 32 * 2 * 2)
        out[f"mfma_fp32_loop_tflops_{w}_waves_per_simd"] = round(flops / s / 1e12, 1)
    # the same loop with v_fma_f32 (kind 0) or LDS reads (kind 1) after every MFMA, at 2
    # waves per SIMD: the drop shows whether the instruction issues beside the matrix core
    for kind, name in ((0, "valu"), (1, "lds_read")):
        res = {}
        for per in (1, 2, 4, 8):
            blocks = cus * 2
            s = timed(lambda: _lib.call("tagi_probe_mfma_mix", buf.data_ptr(), blocks, iters, kind, per, st), 20)
            res[per] = round(blocks * 4 * iters * 4 * (32 * 32 * 2 * 2) / s / 1e12, 1)
        out[f"mfma_fp32_tflops_with_{name}_per_mfma"] = res
    n = (1 << 30) // 4
    src = torch.ones(n, device=dev)
    dst = torch.empty_like(src)
    s = timed(lambda: dst.copy_(src), 10)
    out["copy_1gib_gbs_read_plus_write"] = round(2 * (1 << 30) / s / 1e9, 1)
    # the engine's own streaming kernels (float4, 4 loads in flight per lane), over a sweep
    # of grid sizes: copy (read + write) and read-only
    part = torch.empty(cus * 64 * 256, device=dev)
    for mode, name, nbytes in ((0, "stream_copy_1gib_gbs_read_plus_write", 2 * (1 << 30)),
                               (1, "stream_read_1gib_gbs", 1 << 30)):
        best = {}
        for per_cu in (2, 4, 8, 16, 32, 64):
            blocks = cus * per_cu
            d = dst if mode == 0 else part
            s = timed(lambda: _lib.call("tagi_probe_stream", src.data_ptr(), d.data_ptr(), n, blocks, mode, st), 10)
            best[per_cu] = round(nbytes / s / 1e9, 1)
        out[name] = max(best.values())
        out[name + "_by_blocks_per_cu"] = best
    out["stream_variants"] = measure_stream_variants(dev, src, dst, part, n, cus, st)
    del src, dst, part
    torch.backends.cuda.matmul.allow_tf32 = False
    a = torch.randn(8192, 8192, device=dev)
    b = torch.randn(8192, 8192, device=dev)
    s = timed(lambda: torch.matmul(a, b), 5)
    out["torch_matmul_fp32_8192_tflops"] = round(2 * 8192**3 / s / 1e12, 1)
    return out


def measure_stream_variants(dev, src, dst, part, n, cus, st) -> dict:
    """HBM streaming forms (tagi_probe_stream_variant) over 1 GiB: copy (read + write),
    read-only and write-only; 4, 8 or 16 float4 per lane in flight; nontemporal loads
    and/or stores; grid-stride or one contiguous chunk per block; 8, 32 and 128 blocks of
    256 threads per CU. GB/s of every form, and the best per mode."""
    import torch

    from triton_tagi_amd import _lib

    res = {}
    names = {0: "copy", 1: "read", 2: "write"}
    nbytes = {0: 2 * n * 4, 1: n * 4, 2: n * 4}
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for mode in (0, 1, 2):
        d, dn = (part, part.numel()) if mode == 1 else (dst, dst.numel())
        for unroll in (4, 8, 16):
            for flags in range(8):
                for per_cu in (8, 32, 128):
                    blocks = cus * per_cu
                    if mode == 1 and blocks * 256 > dn:
                        continue

                    def go():
                        _lib.call("tagi_probe_stream_variant", src.data_ptr(), d.data_ptr(), n, dn, blocks, mode,
                                  unroll, flags, st)

                    go()
                    ev0.record()
                    for _ in range(5):
                        go()
                    ev1.record()
                    ev1.synchronize()
                    s = ev0.elapsed_time(ev1) / 1e3 / 5
                    key = (f"{names[mode]} u{unroll} {'ntld' if flags & 1 else 'ld'} {'ntst' if flags & 2 else 'st'} "
                           f"{'chunk' if flags & 4 else 'stride'} {per_cu}/cu")
                    res[key] = round(nbytes[mode] / s / 1e9, 1)
    best = {}
    for mode in names.values():
        k = max((k for k in res if k.startswith(mode)), key=lambda k: res[k])
        best[mode] = {"form": k, "gbs": res[k]}
    return {"best": best, "all": res}


def linear_bench(args) -> dict:
    """Linear microbenchmark: per shape, W warm-up then K timed steps of forward moments,
    backward deltas (input deltas and parameter deltas) and the capped update. As in
    Sequential.step, the update is applied by the kernel that forms the parameter deltas
    (update_in_backward); the layer's update() afterwards finds nothing left to do. The
    parameter deltas are applied without being stored (keep_deltas=False): the step's
    result is the updated parameters, the same bits as with the deltas stored."""
    import torch

    from triton_tagi_amd import workloads
    from triton_tagi_amd.update.in_backward import update_in_backward
    from triton_tagi_amd.update.parameters import get_cap_factor

    shapes, total_flops, total_s = [], 0.0, 0.0
    for (B, K, N) in workloads.LINEAR_SHAPES:
        layer, ma, Sa, dmz, dSz = workloads.linear_microbench(B, K, N)
        cap = get_cap_factor(B)

        def step():
            layer.forward(ma, Sa)
            with update_in_backward(cap, keep_deltas=False):
                layer.backward(dmz, dSz)
            layer.update(cap)

        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / args.steps
        flops = 7 * 2.0 * B * K * N
        total_flops += flops
        total_s += dt
        shapes.append({"batch": B, "in": K, "out": N, "ms_per_step": round(dt * 1e3, 4),
                       "tflops": round(flops / dt / 1e12, 2), "mfma_frac": round(flops / dt / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4)})
        del layer, ma, Sa, dmz, dSz
    return {"tflops": total_flops / total_s / 1e12, "ms": total_s * 1e3, "shapes": shapes}


def heads_bench(args) -> dict:
    """Bandwidth of the output-head and extra-layer kernels at sizes where HBM bounds them.
    Each case: W warm-up then K timed calls on the live HIP-event timer; algorithmic bytes
    per call (each tensor read or written once) over the measured kernel time."""
    import torch

    import triton_tagi_amd as tt
    from triton_tagi_amd import _lib
    from triton_tagi_amd.update.observation import compute_innovation, hrc_innovation

    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(0)

    def rnd(*shape, lo=None):
        t = torch.randn(*shape, device=dev, generator=g)
        return t.abs() + lo if lo is not None else t

    cases = []
    # MaxPool2D 3x3 s2 p1 over a ResNet-stem-sized activation, channels-last
    x = rnd(128, 64, 64, 64).contiguous(memory_format=torch.channels_last)
    xs = rnd(128, 64, 64, 64, lo=0.01).contiguous(memory_format=torch.channels_last)
    mp = tt.MaxPool2D(3, 2, 1)
    out, _ = mp.forward(x, xs)
    dmo, dso = torch.randn_like(out), -torch.rand_like(out)
    cases.append(("maxpool", "MaxPool2D 3x3/2 pad 1 fwd+bwd, (128,64,64,64) channels-last",
                  lambda: (mp.forward(x, xs), mp.backward(dmo, dso))))
    # LayerNorm fwd+bwd over 16384 x 1024 rows
    ln = tt.LayerNorm(1024, device=dev)
    la, ls = rnd(16384, 1024), rnd(16384, 1024, lo=0.01)
    ldm, lds = torch.randn_like(la), -torch.rand_like(la)
    ln.forward(la, ls)
    cases.append(("layernorm", "LayerNorm(1024) fwd+bwd, 16384 rows", lambda: (ln.forward(la, ls), ln.backward(ldm, lds))))
    # EvenSoftplus forward, 32 M elements
    es = tt.EvenSoftplus(1 << 24)
    em, eS = rnd(1 << 25), rnd(1 << 25, lo=0.01)
    cases.append(("softplus", "EvenSoftplus fwd, 2^25 elements", lambda: es.forward(em, eS)))
    # heteroscedastic innovation, 16 M observations (32 M outputs)
    hy = rnd(1 << 24)
    hm, hv = rnd(1 << 25), rnd(1 << 25, lo=0.05)
    hm[1::2] = hm[1::2].abs() + 0.1
    cases.append(("innovation", "heteroscedastic innovation, 2^24 observations",
                  lambda: compute_innovation(hy, hm, hv, 0.0)))
    # HRC sparse innovation, 2^20 rows of an 11-node tree (10 classes)
    hrc = tt.class_to_obs(10)
    rm, rS = rnd(1 << 20, hrc.len), rnd(1 << 20, hrc.len, lo=0.01)
    lab = torch.randint(0, 10, (1 << 20,), device=dev, generator=g)
    cases.append(("innovation", "HRC sparse innovation (labels), 2^20 rows x 11 nodes",
                  lambda: hrc_innovation(rm, rS, lab, hrc, 0.05)))
    cases.append(("innovation", "HRC class probabilities + predicted labels, 2^20 rows x 10 classes",
                  lambda: tt.get_predicted_labels(rm, rS, hrc)))
    res = []
    for fam, desc, fn in cases:
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        _lib.prof_begin([fam])
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        d = _lib.prof_end()[fam]
        gbs = d["bytes"] / (d["ms"] / 1e3) / 1e9
        res.append({"kernel": desc, "family": fam, "us_per_call": round(1e3 * d["ms"] / args.steps, 2),
                    "alg_bytes_per_call": round(d["bytes"] / args.steps), "gbs": round(gbs, 1),
                    "hbm_frac": round(gbs / PEAK_HBM_GBS, 4)})
        log(f"[bench] {desc}: {res[-1]['us_per_call']} us, {res[-1]['gbs']} GB/s")
    return {"cases": res, "bytes": sum(r["alg_bytes_per_call"] for r in res),
            "us": sum(r["us_per_call"] for r in res)}


def load_traffic(workload: str, family: str):
    p = ROOT / "profiles" / "traffic.json"
    if not p.exists():
        return None
    try:
        d = json.loads(p.read_text())
        return d.get(workload, {}).get(family)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="resnet18", choices=sorted(WORKLOAD_DESC))
    ap.add_argument("--batch", type=int, default=None)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time replays of a HIP graph of the step (Sequential.capture_step) instead of eager "
                         "steps; the roofline then comes from the warm-up steps' live timer")
    ap.add_argument("--no-overlap", action="store_true",
                    help="queue the parameter-delta GEMMs on the step's own stream instead of a side stream")
    ap.add_argument("--ceilings", action="store_true",
                    help="print measured MFMA / copy / vendor-GEMM ceilings as one JSON line and exit")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="before warm-up, run one device copy of this many MiB (a known-size kernel for "
                         "calibrating the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this engine runs on one GPU; --gpus {args.gpus} is not supported "
              "(the step shards over the batch only in the design notes, no multi-GPU path is built)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from triton_tagi_amd import _lib, workloads

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = "cuda:0"
    if args.ceilings:
        log("[bench] measuring ceilings")
        print(json.dumps({"ceilings": measure_ceilings(dev)}), flush=True)
        return
    if args.workload == "linear":
        log("[bench] Linear microbenchmark")
        r = linear_bench(args)
        print(json.dumps({
            "metric": "TAGI Linear microbench step (fwd+bwd+update) TFLOP/s, 7 x 2MKN flops per shape",
            "value": round(r["tflops"], 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["ms"], 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32", "data": "synthetic (seeded moments and priors as described in config)",
            "config": {"workload": WORKLOAD_DESC["linear"], "parallelism": "single GPU"},
            "roofline": {"bound": "mfma", "achieved": round(r["tflops"], 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(r["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4), "traffic": None},
            "cpu_baseline": None, "shapes": r["shapes"]}), flush=True)
        return
    if args.workload == "heads":
        log("[bench] output-head and extra-layer kernels")
        r = heads_bench(args)
        agg = r["bytes"] / (r["us"] / 1e6) / 1e9
        top = max(r["cases"], key=lambda c: c["us_per_call"])
        print(json.dumps({
            "metric": "TAGI output-head / extra-layer kernels, aggregate algorithmic GB/s",
            "value": round(agg, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": round(r["us"] / 1e3, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "fp32", "data": "synthetic (seeded moments, labels)",
            "config": {"workload": WORKLOAD_DESC["heads"], "parallelism": "single GPU"},
            "roofline": {"bound": "hbm", "kernel": top["kernel"], "achieved": top["gbs"], "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": top["hbm_frac"], "traffic": None},
            "cpu_baseline": None, "cases": r["cases"]}), flush=True)
        return
    log(f"[bench] building {args.workload} on {dev}")
    w = workloads.build(args.workload, device=dev, batch=args.batch)
    net, x, y, sv = w.net, w.x, w.y, w.sigma_v
    if args.no_overlap:
        net.overlap_param_deltas = False

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] calibration copy of {args.copy_calibration_mib} MiB done")
        del src, dst

    log(f"[bench] warmup {args.warmup} steps (all kernel families timed after the first)")
    fams, prof_steps = {}, 0
    for i in range(args.warmup):
        if i == 1 or (i == 0 and args.warmup == 1):
            torch.cuda.synchronize()
            _lib.prof_begin()
        w.step()
        prof_steps += i >= 1 or args.warmup == 1
    torch.cuda.synchronize()
    if prof_steps:
        fams = _lib.prof_end()
    mfma = {f: v for f, v in fams.items() if f in MFMA_FAMILIES}
    # the dominant kernel: the family with the most algorithmic MFMA work per step (its
    # measured time can include a side stream's kernels sharing the GPU; the forward
    # families, which carry the most work, run alone)
    dom = max(mfma, key=lambda f: mfma[f]["flops"]) if mfma else None

    # The live timer brackets each launch of the dominant family with two HIP events; an
    # event record holds the queue for a few microseconds, so it runs on the last few
    # timed steps only (same shapes every step) instead of inflating all of them.
    timer_steps = min(args.steps, TIMER_STEPS)
    if args.graph:
        log("[bench] recording the step into a HIP graph (one more eager step)")
        graph = net.capture_step_hrc(x, y, w.hrc, sv) if w.hrc is not None else net.capture_step(x, y, sv)
        torch.cuda.synchronize()
        log(f"[bench] timing {args.steps} graph replays")
        t0 = time.perf_counter()
        for i in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        # kernels inside a graph carry no per-launch events: use the warm-up steps' timer
        timed = {dom: fams[dom]} if dom else {}
        timer_steps = max(prof_steps, 1)
    else:
        log(f"[bench] timing {args.steps} steps (timer on {dom or 'no family'} for the last {timer_steps})")
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            if dom and i == args.steps - timer_steps:
                _lib.prof_begin([dom])
            w.step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        timed = _lib.prof_end() if dom else {}
    elapsed = t1 - t0
    ms_per_step = 1e3 * elapsed / args.steps
    value = w.batch * args.steps / elapsed

    roofline = None
    if dom and dom in timed:
        d = timed[dom]
        per_launch_s = d["ms"] / 1e3 / d["launches"]
        flops_per_launch = d["flops"] / d["launches"]
        bytes_per_launch = d["bytes"] / d["launches"]
        # the bound is set by the kernel's algorithmic intensity against the ridge point
        # (157.3 TFLOP/s / 8 TB/s = 19.7 flop/B): products with a short reduction (the
        # attention score products, K = head_dim) are bound by moving their outputs
        hbm_bound = bytes_per_launch > 0 and flops_per_launch / bytes_per_launch < (
            PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9))
        if hbm_bound:
            achieved, peak, unit = bytes_per_launch / per_launch_s / 1e9, PEAK_HBM_GBS, "GB/s"
        else:
            achieved, peak, unit = flops_per_launch / per_launch_s / 1e12, PEAK_FP32_MFMA_TFLOPS, "TFLOP/s"
        roofline = {
            "bound": "hbm" if hbm_bound else "mfma",
            "kernel": dom,
            "achieved": round(achieved, 2),
            "peak": peak,
            "unit": unit,
            "frac": round(achieved / peak, 4),
            "traffic": load_traffic(args.workload, dom),
            "launches_per_step": d["launches"] / timer_steps,
            "timer_steps": timer_steps,
            "avg_launch_us": round(per_launch_s * 1e6, 2),
            "flops_per_launch": round(flops_per_launch),
            "alg_bytes_per_launch": round(bytes_per_launch),
            "alg_flop_per_byte": round(flops_per_launch / bytes_per_launch, 1) if bytes_per_launch else None,
        }
    breakdown = {}
    nps = max(prof_steps, 1)
    gpu_ms = sum(v["ms"] for v in fams.values())
    for f, v in sorted(fams.items(), key=lambda kv: -kv[1]["ms"]):
        e = {"ms_per_step": round(v["ms"] / nps, 4), "launches_per_step": v["launches"] / nps}
        if v["flops"]:
            e["tflops"] = round(v["flops"] / (v["ms"] / 1e3) / 1e12, 2)
            e["mfma_frac"] = round(e["tflops"] / PEAK_FP32_MFMA_TFLOPS, 4)
        elif v["bytes"]:
            e["gbs"] = round(v["bytes"] / (v["ms"] / 1e3) / 1e9, 1)
            e["hbm_frac"] = round(e["gbs"] / PEAK_HBM_GBS, 4)
        breakdown[f] = e

    cpu = None
    if not args.no_cpu_baseline:
        log(f"[bench] cpu baseline (oracle fp32, batch {w.batch})")
        cpu = cpu_baseline(args.workload, w.batch)

    out = {
        "metric": METRIC if args.workload == "resnet18" else
        f"TAGI step samples/sec (fwd+bwd+update) {args.workload} b{w.batch} fp32; % MFMA/HBM peak",
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded inputs, one-hot targets or class labels, random-init priors of the architecture)",
        "config": {"workload": WORKLOAD_DESC[args.workload], "global_batch": w.batch, "parallelism": "single GPU",
                   "launch": "hip graph replay" if args.graph else "eager",
                   "param_deltas": "side stream" if net.overlap_param_deltas else "step stream"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernel_ms_per_step_warmup": round(gpu_ms / nps, 4),
        # the family with the most GPU time per step (with the side stream, the parameter-
        # delta families' time includes sharing the GPU with the input-delta chain)
        "top_family_by_time": next(iter(breakdown), None),
        "families_warmup": breakdown,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
