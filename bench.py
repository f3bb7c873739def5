"""MoE-layer throughput on one MI355X, with the dominant kernel's roofline and a CPU baseline.

A step is one pass of the routed MoE layer (router gemm -> topk_softmax -> moe_sort ->
gather_gemm -> route_gemm -> moe_unpermute, through the library's C entries) over one batch of
synthetic tokens already resident in HBM. The default workload is BASELINE.json configs[1]:
Qwen3-30B-A3B-shaped layer, bf16, 64-token decode (H=2048, E=128, top-8, I=768), weights
~N(0, 0.02) and activations ~N(0, 1) from a seed (near-uniform routing).

Prints ONE JSON line. `value` is tokens/s of the whole layer; `roofline` is the dominant kernel's
achieved algorithmic GB/s (decode) or TFLOP/s (prefill) from HIP events around its launches inside
the timed region; `cpu_baseline` is the CPU oracle's restatement of the reference CPU formulas
(`Fused::cpu`, crates/nn/src/functional/moe.rs) on the same inputs, timed on this host.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "uniserve-v1_amd"))

METRIC = "MoE-layer tokens/s + % of HBM (decode) / MFMA (prefill) roofline, 1 GPU"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
# Dense peaks; an MXFP4 x MXFP8 scaled MFMA runs at the fp8 rate (its B operand is e4m3).
MFMA_PEAK_TFLOPS = {"bf16": 2500.0, "f8e4m3": 5000.0, "f4e2m1": 5000.0}

CONFIGS = {
    # name: tokens, hidden, experts, top, intermediate, weights, zipf routing
    "30b-decode-bf16": (64, 2048, 128, 8, 768, "bf16", False),
    "30b-prefill-bf16": (8192, 2048, 128, 8, 768, "bf16", True),
    "30b-decode-fp8": (64, 2048, 128, 8, 768, "f8e4m3", False),
    "30b-prefill-fp8": (8192, 2048, 128, 8, 768, "f8e4m3", True),
    "235b-prefill-fp8": (4096, 4096, 128, 8, 1536, "f8e4m3", True),
    "235b-decode-fp8": (1, 4096, 128, 8, 1536, "f8e4m3", False),
    "30b-decode-mx": (64, 2048, 128, 8, 768, "f4e2m1", False),
    "30b-prefill-mx": (8192, 2048, 128, 8, 768, "f4e2m1", True),
    "235b-decode-mx": (1, 4096, 128, 8, 1536, "f4e2m1", False),
    "235b-prefill-mx": (4096, 4096, 128, 8, 1536, "f4e2m1", True),
}


def parse():
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=200)
    parser.add_argument("--warmup", type=int, default=20)
    parser.add_argument("--config", default="30b-decode-bf16", choices=sorted(CONFIGS))
    parser.add_argument("--extra", action="store_true", help="also measure every other BASELINE config")
    parser.add_argument("--also", default="30b-prefill-fp8,30b-prefill-bf16",
                        help="comma-separated configs measured briefly beside the main one (default: the fp8 "
                             "and bf16 prefill targets' config); '' for none")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU-baseline leg")
    parser.add_argument("--cpu-runs", type=int, default=3)
    parser.add_argument("--traffic-summary", metavar="DIR",
                        help="only fold rocprofv3 FETCH_SIZE / WRITE_SIZE passes (DIR/<config>/{fetch,write}, "
                             "DIR/calibration/{fetch,write}, csv) into profiles/hbm_traffic.json")
    parser.add_argument("--copy-calibration", action="store_true",
                        help="only run a plain elementwise copy of 1 GiB in, 1 GiB out (five launches): the "
                             "known-size reference for scaling FETCH_SIZE / WRITE_SIZE counter readings")
    return parser.parse_args()


class Workload:
    """Synthetic weights and tokens of one config, resident on the device."""

    def __init__(self, name, seed=0):
        import torch

        from uniserve_moe import ops
        from uniserve_moe.checkpoint import quantize_blocks_e4m3, quantize_blocks_mxfp4

        self.name = name
        (self.tokens, self.hidden, self.experts, self.top, self.intermediate, self.wdtype,
         self.zipf) = CONFIGS[name]
        device = torch.device("cuda:0")
        g = torch.Generator(device=device).manual_seed(seed)

        def normal(shape, std):
            return (torch.randn(shape, generator=g, device=device) * std).to(torch.bfloat16)

        T, H, E, I = self.tokens, self.hidden, self.experts, self.intermediate
        self.x = normal((T, H), 1.0)
        self.router = normal((E, H), 0.02)
        self.up_gate_bf16 = normal((E, 2 * I, H), 0.02)
        self.down_bf16 = normal((E, H, I), 0.02)
        self.bias = None
        if self.zipf:
            self.bias = (-1.1 * torch.log(torch.arange(E, device=device, dtype=torch.float32) + 1.0)).contiguous()
        self.scales = {}
        if self.wdtype == "f8e4m3":
            # Setup, not timed: 128 x 128 block-scaled e4m3 (scale = blockmax / 448).
            self.up_gate, s1 = quantize_blocks_e4m3(self.up_gate_bf16)
            self.down, s2 = quantize_blocks_e4m3(self.down_bf16)
            self.scales = dict(up_gate_scales=s1, down_scales=s2)
        elif self.wdtype == "f4e2m1":
            # Setup, not timed: OCP MXFP4 (E2M1 pairs, an E8M0 scale per 32 along K).
            # Scales converted once, at load, to the stage-major layout the prefill kernel fetches
            # a stage of 256 rows from as one run (the decode kernel reads either).
            self.up_gate, s1 = quantize_blocks_mxfp4(self.up_gate_bf16)
            self.down, s2 = quantize_blocks_mxfp4(self.down_bf16)
            self.scales = dict(up_gate_scales=ops.mx_stage_major_scales(s1), down_scales=ops.mx_stage_major_scales(s2),
                               scale_layout="stage")
            self.row_major_scales = (s1, s2)
        else:
            self.up_gate, self.down = self.up_gate_bf16, self.down_bf16
        self.layer = ops.MoeLayer(H, E, self.top, I, T, weight_dtype=self.wdtype)
        self.out = torch.empty((T, H), dtype=torch.bfloat16, device=device)

    def step(self):
        return self.layer(self.x, self.router, self.up_gate, self.down, out=self.out,
                          router_bias=self.bias, **self.scales)


def measure(w, steps, warmup):
    """Times `steps` layer calls (after `warmup`), and the FC1 / FC2 kernels inside them."""
    import torch

    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        w.step()
    torch.cuda.synchronize()
    # The whole layer: K back-to-back calls bracketed by synchronisations.
    start = time.perf_counter()
    for _ in range(steps):
        w.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - start

    # The dominant kernels, launched exactly as the layer launches them (its own step entry, same
    # arguments and workspace), timed with events on their stream.
    fc = {"gather_gemm": [], "route_gemm": []}
    fc1 = lambda: w.layer.step("gather")  # noqa: E731
    fc2 = lambda: w.layer.step("route")  # noqa: E731
    for _ in range(max(3, warmup // 4)):
        fc1()
        fc2()
    torch.cuda.synchronize()
    for _ in range(steps):
        for name, fn in (("gather_gemm", fc1), ("route_gemm", fc2)):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            fc[name].append((a, b))
    torch.cuda.synchronize()
    kernel_ms = {name: sum(a.elapsed_time(b) for a, b in pairs) / len(pairs) for name, pairs in fc.items()}
    return elapsed, kernel_ms


def graph_timing(w, steps, calls=20):
    """The same layer calls replayed from a captured HIP graph (`calls` per replay, at least three
    replays): the device's own time per call, free of the host's per-call launch work. The first
    two replays' outputs are checked against the eager call's, bit for bit."""
    import torch

    w.step()
    torch.cuda.synchronize()
    eager = w.out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(calls):
                w.step()
    torch.cuda.synchronize()
    replays = max(3, steps // calls)
    for _ in range(2):
        w.out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(w.out, eager):
            raise RuntimeError("graph replay of the layer differs from the eager call")
    start = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    return (time.perf_counter() - start) / (replays * calls)


def algorithmic(w):
    """Algorithmic bytes and flops of the layer and of FC1, from the run's own routing."""
    import torch

    ids = w.layer.view("ids", torch.int32, (w.tokens, w.top)).cpu()
    touched = int(torch.unique(ids).numel())
    routes = w.tokens * w.top
    # Bytes per weight element (MXFP4: half a byte plus an E8M0 byte per 32 elements).
    elem = {"bf16": 2, "f8e4m3": 1, "f4e2m1": 0.5 + 1 / 32}[w.wdtype]
    H, I, E, T = w.hidden, w.intermediate, w.experts, w.tokens
    scale_bytes = 0
    if w.wdtype == "f8e4m3":
        scale_bytes = touched * ((2 * I // 128) * (H // 128) + (H // 128) * (I // 128)) * 4
    layer_bytes = int(touched * 3 * H * I * elem) + scale_bytes + T * H * 2 * 2 + H * E * 2
    layer_flops = 2 * routes * 3 * H * I + 2 * T * H * E
    act_elem = {"bf16": 2, "f8e4m3": 1, "f4e2m1": 1 + 1 / 32}[w.wdtype]
    # FC1 writes the gated rows in bf16, or (e4m3 prefill shapes) as e4m3 codes with a scale per
    # 128 columns.
    gated_elem = 1 + 4 / 128 if w.wdtype == "f8e4m3" and w.layer.views.route_scales else 2
    fc1_bytes = int(touched * 2 * I * H * elem + T * H * act_elem + routes * I * gated_elem)
    if w.wdtype == "f8e4m3":
        fc1_bytes += touched * (2 * I // 128) * (H // 128) * 4 + T * (H // 128) * 4
    fc1_flops = 2 * routes * 2 * I * H
    return dict(touched=touched, layer_bytes=layer_bytes, layer_flops=layer_flops, fc1_bytes=fc1_bytes,
                fc1_flops=fc1_flops)


def cpu_baseline(w, runs):
    """The CPU oracle (tests/oracle_lib.py over oracle/libmoe_oracle.so) on the same layer inputs."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "tests"))
    import oracle_lib

    def bits(t):
        return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)

    x, router = bits(w.x), bits(w.router)
    if w.wdtype in ("f8e4m3", "f4e2m1"):
        up_gate, down = w.up_gate.cpu().numpy(), w.down.cpu().numpy()
        if w.wdtype == "f4e2m1":
            s1, s2 = (t.cpu().numpy() for t in w.row_major_scales)
        else:
            s1 = w.scales["up_gate_scales"].cpu().numpy()
            s2 = w.scales["down_scales"].cpu().numpy()
    else:
        up_gate, down, s1, s2 = bits(w.up_gate), bits(w.down), None, None
    oracle_lib.moe_layer(x[:1], router, up_gate, down, w.top, up_gate_scales=s1, down_scales=s2)  # warm
    times = []
    threads = 1
    for _ in range(runs):
        t0 = time.perf_counter()
        _, _, _, threads = oracle_lib.moe_layer(x, router, up_gate, down, w.top, up_gate_scales=s1, down_scales=s2)
        times.append(time.perf_counter() - t0)
    median = sorted(times)[len(times) // 2]
    return {"value": round(w.tokens / median, 2), "unit": "tokens/s", "cores": int(threads), "kind": "port",
            "sample": f"the whole {w.name} layer ({w.tokens} tokens), median of {runs} runs "
                      f"({median * 1e3:.1f} ms each): C restatement of the reference's Fused::cpu formulas, "
                      f"OpenMP over {threads} threads"}


def measured_traffic(name):
    """HBM bytes per gather_gemm launch for this config, from the committed counter summary
    (FETCH_SIZE and WRITE_SIZE passes scaled by a copy kernel of known size), or None."""
    path = ROOT / "profiles" / "hbm_traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get("configs", {}).get(name, {}).get("gather_gemm")
    return None if entry is None else entry["hbm_bytes"]


def counter_means(directory, counter):
    """Mean per-dispatch value of `counter` per kernel name, over every counter CSV under `directory`."""
    import csv

    sums, counts = {}, {}
    for path in Path(directory).rglob("*counter_collection.csv"):
        with open(path) as handle:
            for row in csv.DictReader(handle):
                if row["Counter_Name"] != counter:
                    continue
                key = row["Kernel_Name"]
                sums[key] = sums.get(key, 0.0) + float(row["Counter_Value"])
                counts[key] = counts.get(key, 0) + 1
    return {key: sums[key] / counts[key] for key in sums}


def traffic_summary(directory):
    """HBM bytes per launch of the grouped products of each config: FETCH_SIZE and WRITE_SIZE (KiB
    per dispatch) scaled so that a plain copy of 1 GiB in / 1 GiB out reads exactly its bytes."""
    root = Path(directory)
    calib_fetch = max(counter_means(root / "calibration" / "fetch", "FETCH_SIZE").values())
    calib_write = max(counter_means(root / "calibration" / "write", "WRITE_SIZE").values())
    gib_kib = float(1 << 20)
    fetch_scale, write_scale = gib_kib / calib_fetch, gib_kib / calib_write
    import re

    products = {"gather_gemm": "true", "route_gemm": "false"}
    pattern = re.compile(r"((?:stream|prefill|tiled|pair|quarter)\w*)(?:<([^<>]*)>)?\(")
    configs = {}
    for name in CONFIGS:
        if not (root / name).exists():
            continue
        fetch = counter_means(root / name / "fetch", "FETCH_SIZE")
        write = counter_means(root / name / "write", "WRITE_SIZE")
        entry = {}
        for product, gated in products.items():
            def gated_flag(match):  # prefill_kernel / pair_kernel<format, gated>; the others <gated, ...>
                if match.group(2) is None:  # quarter_kernel: FC1 only
                    return "true"
                args = [a.strip() for a in match.group(2).split(",")]
                return args[-1] if match.group(1).startswith(("prefill", "pair")) else args[0]

            found = [(k, m) for k, m in ((k, pattern.search(k)) for k in fetch) if m and gated_flag(m) == gated]
            if not found:
                continue
            kernel, match = found[0]
            f, wr = fetch[kernel], write.get(kernel, 0.0)
            args = "" if match.group(2) is None else f"<{match.group(2).replace('uniserve::', '')}>"
            entry[product] = {"kernel": f"{match.group(1)}{args}",
                              "fetch_KiB": round(f, 1),
                              "write_KiB": round(wr, 1),
                              "hbm_bytes": int(f * 1024 * fetch_scale + wr * 1024 * write_scale)}
        configs[name] = entry
    summary = {"method": "rocprofv3 --pmc FETCH_SIZE, then --pmc WRITE_SIZE (KiB per dispatch, averaged over the "
                         "run's dispatches of the kernel), scaled by the readings for a plain elementwise copy of "
                         "1 GiB in / 1 GiB out (bench.py --copy-calibration)",
               "fetch_scale": round(fetch_scale, 4), "write_scale": round(write_scale, 4), "configs": configs}
    (ROOT / "profiles" / "hbm_traffic.json").write_text(json.dumps(summary, indent=1) + "\n")
    print(json.dumps(summary))


def run_config(name, steps, warmup, with_cpu, cpu_runs):
    w = Workload(name)
    elapsed, kernel_ms = measure(w, steps, warmup)
    graph_s = graph_timing(w, steps)
    alg = algorithmic(w)
    ms_per_step = elapsed / steps * 1e3
    tokens_per_s = w.tokens * steps / elapsed
    decode = not w.zipf and w.tokens <= 256
    fc1_s = kernel_ms["gather_gemm"] * 1e-3
    if decode:
        achieved = alg["fc1_bytes"] / fc1_s / 1e9
        roofline = {"kernel": "gather_gemm (FC1 + SiLU)", "bound": "hbm", "achieved": round(achieved, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(name),
                    "avg_launch_us": round(kernel_ms["gather_gemm"] * 1e3, 2)}
    else:
        achieved = alg["fc1_flops"] / fc1_s / 1e12
        peak = MFMA_PEAK_TFLOPS[w.wdtype]
        roofline = {"kernel": "gather_gemm (FC1 + SiLU)", "bound": "mfma", "achieved": round(achieved, 1),
                    "peak": peak, "unit": "TFLOP/s", "frac": round(achieved / peak, 4), "traffic": measured_traffic(name),
                    "avg_launch_us": round(kernel_ms["gather_gemm"] * 1e3, 2)}
    layer = {
        "ms_per_step": round(ms_per_step, 4),
        "tokens_per_s": round(tokens_per_s, 1),
        "layer_GBps": round(alg["layer_bytes"] / (ms_per_step * 1e-3) / 1e9, 1),
        "layer_TFLOPs": round(alg["layer_flops"] / (ms_per_step * 1e-3) / 1e12, 2),
        "layer_hbm_frac": round(alg["layer_bytes"] / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "layer_mfma_frac": round(alg["layer_flops"] / (ms_per_step * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS[w.wdtype], 4),
        "touched_experts": alg["touched"],
        "route_gemm_us": round(kernel_ms["route_gemm"] * 1e3, 2),
        "gather_gemm_us": round(kernel_ms["gather_gemm"] * 1e3, 2),
        # The same calls replayed from a HIP graph (not `value`: the eager calls are).
        "graph_ms_per_step": round(graph_s * 1e3, 4),
        "graph_tokens_per_s": round(w.tokens / graph_s, 1),
    }
    cpu = cpu_baseline(w, cpu_runs) if with_cpu else None
    return w, ms_per_step, tokens_per_s, roofline, layer, cpu


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU: every box here has one MI355X and the layer "
                          "holds all experts on it (expert-parallel sharding is a design note, not a path). "
                          "Run with --gpus 1."}))
        sys.exit(2)
    if args.traffic_summary:
        traffic_summary(args.traffic_summary)
        return
    import torch

    if args.copy_calibration:
        source = torch.ones(1 << 28, dtype=torch.float32, device="cuda")
        target = torch.empty_like(source)
        for _ in range(5):
            torch.neg(source, out=target)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": source.numel() * 4, "bytes_written": target.numel() * 4,
                                               "launches": 5, "kernel": "elementwise neg"}}))
        return

    w, ms_per_step, tokens_per_s, roofline, layer, cpu = run_config(
        args.config, args.steps, args.warmup, not args.no_cpu, args.cpu_runs)
    line = {
        "metric": METRIC,
        "value": round(tokens_per_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bf16": "bf16", "f8e4m3": "fp8-e4m3 (bf16 out)",
                  "f4e2m1": "mxfp4 weights x mxfp8 activations (bf16 out)"}[w.wdtype],
        "data": "synthetic (seeded N(0,1) tokens, N(0,0.02) weights)",
        "config": {"workload": f"Qwen3-MoE layer {args.config}", "tokens": w.tokens, "hidden": w.hidden,
                   "experts": w.experts, "top": w.top, "intermediate": w.intermediate,
                   "routing": "zipf(1.1) bias" if w.zipf else "near-uniform", "parallelism": "single GPU, all experts resident"},
        "roofline": roofline,
        "layer": layer,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(0),
    }
    others = list(CONFIGS) if args.extra else [name for name in args.also.split(",") if name]
    extra = {}
    for name in others:
        if name == args.config:
            continue
        if name not in CONFIGS:
            raise SystemExit(f"unknown config {name!r}")
        del w
        torch.cuda.empty_cache()
        w, ms, tps, roof, lay, _ = run_config(name, max(10, args.steps // 10), max(3, args.warmup // 4), False, 0)
        extra[name] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(tps, 1), "roofline": roof, "layer": lay}
    if extra:
        line["extra"] = extra
    print(json.dumps(line))


if __name__ == "__main__":
    main()
