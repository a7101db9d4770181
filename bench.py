"""MoE-layer throughput of the HIP path on one MI355X, with roofline and CPU baseline.

A "step" is one pass of the routed expert FFN (routing, dispatch, gate_up +
SiLU·mul, down + route weight, rank-ordered combine) over one batch of
synthetic tokens already resident in HBM.  Default workload: the
Qwen3-30B-A3B-shaped layer at batch-64 decode; weights
rotate over 4 banks so the 256 MB MALL cannot hold the layer.  The default
run also measures the same layer at 4096-token prefill and
reports it under "prefill".

Prints ONE JSON line.  The headline `value` / `ms_per_step` time exactly
--steps rotating-bank steps after --warmup.  `timing` adds the reference's
methodology (crates/models/src/components/cuda/fused_moe/validation/timing.rs:
7 rounds, the first discarded, median): rotating and hot banks, eager launches
and HIP-graph replays.  `roofline` describes the dominant kernel of the step
(the fused decode gate_up kernel for decode, the MFMA grouped gate_up for
prefill), timed alone with HIP events on the stream it runs on;
`cpu_baseline` is the C restatement of the reference's f32 CPU path (the
oracle) on a bounded token sample, on this host's cores.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

WORKLOADS = {
    "c2": "c2_30b_a3b_decode",
    "c3": "c3_30b_a3b_prefill",
    "c4": "c4_next_sparse",
    "c5p": "c5_235b_prefill",
    "c5d": "c5_235b_decode",
}


def load_package():
    if "tau_rs_amd" in sys.modules:
        return sys.modules["tau_rs_amd"]
    pkg = os.path.join(ROOT, "tau.rs_amd")
    spec = importlib.util.spec_from_file_location("tau_rs_amd", os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["tau_rs_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--banks", type=int, default=0, help="weight banks to rotate (0 = auto)")
    ap.add_argument("--tile-rows", type=int, default=0, help="override the library's row-block choice")
    ap.add_argument("--tokens", type=int, default=0, help="run the workload's layer at this many tokens")
    ap.add_argument("--weight-layout", choices=("auto", "row_major", "frag16"), default="auto",
                    help="expert weight layout held by the runner (auto: FRAG16 when the shape allows)")
    ap.add_argument("--with-norm", action="store_true",
                    help="time the decoder's feed-forward half: fused residual add + centered RMSNorm, then the "
                         "MoE layer with the final residual add fused into its combine")
    ap.add_argument("--with-router", action="store_true",
                    help="start the step from hidden states: the router projection and routing "
                         "(tau_launch_moe_router_route_ex), then the layer from those routes")
    ap.add_argument("--shared-apart", action="store_true",
                    help="run a shared expert with its own launches instead of folded into the routed schedule")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true",
                    help="with the default workload, skip the c3 prefill sub-object")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP-graph replay timings")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (HBM counter calibration under rocprofv3 --pmc)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


class Layer:
    """One workload: inputs, rotating weight banks and a dispatch workspace."""

    def __init__(self, tau, torch, shape, banks, tile_rows=0, weight_layout="auto", with_norm=False,
                 with_router=False, shared_apart=False):
        self.tau, self.torch, self.shape = tau, torch, shape
        self.data = tau.inputs.make_layer(shape)
        d = self.data
        # A gated shared expert with the experts' intermediate size runs as expert E
        # of the routed schedule (every token takes it at rank K, weight sigmoid(x . w_s)).
        self.folded = bool(shape.shared_intermediate) and shape.shared_intermediate == shape.intermediate \
            and not shared_apart
        self.experts = shape.experts + (1 if self.folded else 0)   # as launched
        self.top_k = shape.top_k + (1 if self.folded else 0)
        if self.folded:  # router logits then the shared gate logit x . w_s (f32), like the router projection
            gate = d["x"].float() @ d["shared_gate"].float().reshape(-1, 1)
            self.logits_ext = torch.cat([d["logits"].float(), gate], 1).contiguous()
        self.router = None
        if with_router:  # BF16 router weight (+ w_s when folded), f32 bias, logits output
            w, b = d["router"].to(torch.bfloat16), d["bias"]
            if self.folded:
                w = torch.cat([w, d["shared_gate"].reshape(1, -1).to(torch.bfloat16)], 0)
                b = torch.cat([b, torch.zeros(1, device="cuda")])
            self.router = (w.contiguous(), b.contiguous(),
                           torch.empty(shape.tokens, self.experts, dtype=torch.float32, device="cuda"))
        self.norm = None
        if with_norm:  # attention-branch output, norm weight, residual and normalized buffers
            g = torch.Generator(device="cuda").manual_seed(shape.seed + 100)
            x = self.data["x"]
            self.norm = (torch.randn(x.shape, generator=g, device="cuda").to(torch.bfloat16),
                         (torch.randn(shape.hidden, generator=g, device="cuda") * 0.1).to(torch.bfloat16),
                         torch.empty_like(x), torch.empty_like(x))
        cfg = tau.SparseMoeConfig(shape.hidden, shape.intermediate, shape.experts, shape.top_k)
        # The runner prepares the weights once (load time): FRAG16 copies when
        # the shape allows, as a serving deployment would hold them.
        if self.folded:
            gu_all = torch.cat([d["gate_up"], d["shared_gate_up"].unsqueeze(0)], 0)
            dn_all = torch.cat([d["down"], d["shared_down"].unsqueeze(0)], 0)
            self.runner = tau.MoePrefillRunner(cfg, gu_all, dn_all, tile_rows=tile_rows or None,
                                               weight_layout=weight_layout, fold_shared=True)
            del gu_all, dn_all
        else:
            self.runner = tau.MoePrefillRunner(cfg, d["gate_up"], d["down"], tile_rows=tile_rows or None,
                                               weight_layout=weight_layout)
        self.layout = self.runner.layout
        self.shared = None
        if shape.shared_intermediate and not self.folded:  # the shared expert's own launches
            gu_s, dn_s = self.data["shared_gate_up"], self.data["shared_down"]
            lay = tau.ffi.WEIGHTS_ROW_MAJOR
            if self.layout == tau.ffi.WEIGHTS_FRAG16 and shape.shared_intermediate % 64 == 0:
                gu_s, dn_s, lay = tau.ffi.pack_weights(gu_s), tau.ffi.pack_weights(dn_s), tau.ffi.WEIGHTS_FRAG16
            T = shape.tokens
            self.shared = (gu_s, dn_s, self.data["shared_gate"], lay,
                           torch.empty(T, shape.shared_intermediate, dtype=torch.bfloat16, device="cuda"),
                           torch.empty(T, shape.hidden, dtype=torch.bfloat16, device="cuda"))
        self.banks = [(self.runner.gate_up, self.runner.down)]
        for _ in range(banks - 1):
            self.banks.append((self.runner.gate_up.clone(), self.runner.down.clone()))
        self.tile_rows = self.runner.tile_rows_for(shape.tokens)
        self.ws = self.runner.workspace(shape.tokens, self.tile_rows)
        self.out = torch.empty_like(self.data["x"])
        self.receipts = torch.zeros(10, dtype=torch.int32, device="cuda")

    def residual_norm(self, i=0):
        """residual = x + branch (BF16), normalized = centered RMSNorm(residual)."""
        branch, w, res, normed = self.norm
        x = self.data["x"]
        ffi = self.tau.ffi
        ffi.check(ffi.lib().tau_launch_fused_residual_rms_norm(
            ffi.ptr(x), ffi.ptr(branch), ffi.ptr(w), ffi.ptr(res), ffi.ptr(normed), x.shape[0], x.shape[1], 1e-6, 1,
            ffi.stream_ptr(), 16), "fused residual RMSNorm")

    def route_from_hidden(self, i=0, x=None):
        """Router projection (bias fused) and routing into the workspace's routes."""
        w, b, logits = self.router
        x = self.data["x"] if x is None else x
        if self.folded:
            self.tau.ffi.router_route_shared_ex(x, w, b, logits, self.ws["routes"], self.shape.experts,
                                                self.shape.top_k)
        else:
            self.tau.ffi.router_route_ex(x, w, b, logits, self.ws["routes"], self.shape.top_k)

    def project_router(self, i=0):
        """The router projection alone."""
        w, b, logits = self.router
        self.tau.ffi.router_ex(self.data["x"], w, b, logits)

    def step(self, i):
        gu, dn = self.banks[i % len(self.banks)]
        s = self.shape
        x, residual = self.data["x"], None
        if self.norm is not None:
            self.residual_norm()
            x, residual = self.norm[3], self.norm[2]
        logits = self.data["logits"]
        if self.router is not None:
            self.route_from_hidden(x=x)
            logits = None
        elif self.folded:  # routed top-K plus the shared expert at rank K
            self.tau.ffi.routing_shared_ex(self.logits_ext, self.ws["routes"], s.experts, s.top_k)
            logits = None
        # the residual add finishes the block: in the combine, or in the shared combine when there is one
        self.tau.ffi.prefill_ex(x, logits, gu, dn, self.ws, self.out, self.experts,
                                self.top_k, self.tile_rows, receipts=self.receipts, weight_layout=self.layout,
                                residual=residual if self.shared is None else None)
        if self.shared is not None:
            gu_s, dn_s, gate, lay, act, sh = self.shared
            self.tau.ffi.shared_expert_ex(x, gu_s, dn_s, gate, self.out, act, sh, self.out,
                                          weight_layout=lay, residual=residual)

    def decode_path(self):
        """True when the step takes the fused decode path (its own projection kernels)."""
        s = self.shape
        return self.tile_rows == 16 and s.tokens <= 64 and self.experts <= 256 and \
            s.hidden % 64 == 0 and s.intermediate % 64 == 0

    def projection(self, i, which):
        """One launch of the step's gate_up (0) or down (1) kernel over the live
        routes / dispatch, on bank i: the fused decode kernels on the decode
        path, the grouped kernels otherwise."""
        gu, dn = self.banks[i % len(self.banks)]
        s = self.shape
        if which == 0:
            a, w, out = self.data["x"], gu, self.ws["activated"]
        else:
            a, w, out = self.ws["activated"], dn, self.ws["contributions"]
        if self.decode_path():
            self.tau.ffi.decode_projection_ex(a, w, self.ws, out, s.tokens, s.hidden, s.intermediate, self.experts,
                                              self.top_k, which, weight_layout=self.layout)
            return
        self.tau.ffi.grouped_gemm_ex(a, w, self.ws, out, s.tokens, s.hidden, s.intermediate, self.experts, self.top_k,
                                     self.tile_rows, which, weight_layout=self.layout)


def time_events(torch, fn, n, offset=0):
    """Average duration (ms) of n back-to-back launches, HIP events on the launch stream."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(n):
        fn(offset + i)
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / n


def rounds_median(torch, fn, n, rounds):
    """Median over rounds 1.. of the per-round average (round 0 is discarded),
    the methodology of the reference's fused-MoE timing
    (crates/models/src/components/cuda/fused_moe/validation/timing.rs:40-74)."""
    per_round = [time_events(torch, fn, n, offset=r * n) for r in range(rounds)]
    return statistics.median(per_round[1:]), per_round


def graph_of(torch, fn, count):
    """A HIP graph holding fn(0) .. fn(count - 1) (one eager pass first)."""
    for i in range(count):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return graph


def cpu_baseline(layer, seconds):
    """Oracle f32 (restatement of the reference CPU path) on a token sample."""
    sys.path.insert(0, ROOT)
    from oracle import oracle

    s = layer.shape
    sample = s.tokens if s.tokens <= 64 else 256
    f = lambda t: t.float().cpu().numpy()
    x = f(layer.data["x"][:sample])
    lg = f(layer.data["logits"][:sample])
    gu = f(layer.data["gate_up"])
    dn = f(layer.data["down"])
    shared = None
    if s.shared_intermediate:
        shared = (f(layer.data["shared_gate_up"]), f(layer.data["shared_down"]), f(layer.data["shared_gate"]))
    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = nproc
    threads = max(1, min(16, usable))  # a one-GPU box's CPU share
    oracle.set_threads(threads)
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 2000):  # ~`seconds` of CPU work
        t0 = time.perf_counter()
        ids, w = oracle.route(lg, s.top_k)
        routed = oracle.moe(x, ids, w, gu, dn)
        if shared is not None:
            oracle.shared_combine_f32(x, shared[2], oracle.dense_mlp(x, shared[0], shared[1]), routed)
        times.append(time.perf_counter() - t0)
    med = statistics.median(times[1:]) if len(times) > 1 else times[0]
    return {
        "value": sample / med,
        "unit": "tokens/s",
        "cores": threads,
        "nproc": nproc,
        "affinity_cpus": usable,
        "kind": "port",
        "sample": f"{sample} of {s.tokens} tokens of {s.name}, f32 C restatement of the reference CPU path "
                  f"(oracle/moe_oracle.c, OpenMP, {threads} threads), median of {len(times) - 1} passes after "
                  f"1 warm-up, {sum(times):.1f} s of CPU work",
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.txt")


def measured_traffic(workload, kernel, layout):
    """HBM bytes per launch (fetch + write) recorded from rocprofv3 --pmc runs
    in profiles/hbm_traffic.txt (lines: workload kernel fetch write layout), or
    None when not measured for this case."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        parts = line.split()
        if line.startswith("#") or len(parts) != 5:
            continue
        if parts[0] == workload and parts[1] == kernel and parts[4] == layout:
            return int(parts[2]) + int(parts[3])
    return None


def copy_calibration(torch):
    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "launches": 5}), flush=True)


def measure(tau, torch, shape, args, banks, steps, warmup, label):
    """Times one workload: exactly `steps` rotating-bank steps after `warmup`
    (the headline), then the reference's rounds methodology for rotating and
    hot banks, eager and graph-replayed, and the dominant projection alone."""
    layer = Layer(tau, torch, shape, banks, args.tile_rows, args.weight_layout, args.with_norm, args.with_router,
                  args.shared_apart)
    print(f"[bench] {label}: {shape.name} T={shape.tokens} banks={banks} tile_rows={layer.tile_rows}",
          file=sys.stderr, flush=True)
    for i in range(warmup):
        layer.step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_step = time_events(torch, layer.step, steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0

    # Routing facts for the algorithmic work.
    meta = layer.ws["meta"][: 2 * layer.experts + 2].cpu()
    counts = meta[: shape.experts]  # routed experts (a folded shared expert is expert E)
    distinct = int((counts > 0).sum())
    status = int(meta[2 * layer.experts])
    flops, bytes_ = tau.inputs.algorithmic_work(shape, distinct)

    # Rounds (7, the first discarded, median of the rest) of `n` steps each.
    rounds, n = 7, max(10, min(steps, 50))
    hot = lambda i: layer.step(0)
    timing = {"rounds": rounds, "steps_per_round": n, "discarded_rounds": 1}
    timing["rotating_eager_ms"], per_round = rounds_median(torch, layer.step, n, rounds)
    timing["rotating_eager_rounds_ms"] = per_round
    timing["hot_eager_ms"], _ = rounds_median(torch, hot, n, rounds)
    if not args.no_graph:
        g_rot = graph_of(torch, layer.step, len(layer.banks))
        g_hot = graph_of(torch, hot, 1)
        timing["rotating_graph_ms"], _ = rounds_median(torch, lambda i: g_rot.replay(), max(1, n // len(layer.banks)),
                                                       rounds)
        timing["rotating_graph_ms"] /= len(layer.banks)
        timing["hot_graph_ms"], _ = rounds_median(torch, lambda i: g_hot.replay(), n, rounds)
        del g_rot, g_hot

    # Per-projection timing over the live routes / dispatch (one untimed launch
    # each first: code objects load on their first launch), rotating banks.
    n_proj = max(10, steps)
    layer.projection(0, 0)
    layer.projection(0, 1)
    torch.cuda.synchronize()
    ms_gu = time_events(torch, lambda i: layer.projection(i, 0), n_proj)
    ms_dn = time_events(torch, lambda i: layer.projection(i, 1), n_proj)
    T, H, I, K = shape.tokens, shape.hidden, shape.intermediate, shape.top_k
    A = T * layer.top_k  # assignments per launch (a folded shared expert adds T)
    d_launch = distinct + (1 if layer.folded else 0)
    # Algorithmic bytes and FLOPs per launch of each projection.
    gu_bytes = d_launch * 2 * I * H * 2 + T * H * 2 + A * I * 2
    dn_bytes = d_launch * H * I * 2 + A * I * 2 + A * H * 2
    gu_flops, dn_flops = 2 * A * H * 2 * I, 2 * A * I * H
    kernels = {}
    for name, ms, b, f in (("gate_up", ms_gu, gu_bytes, gu_flops), ("down", ms_dn, dn_bytes, dn_flops)):
        kernels[name] = {"us": ms * 1e3, "algorithmic_bytes": b, "algorithmic_flops": f,
                         "GB/s": b / (ms * 1e-3) / 1e9, "TFLOP/s": f / (ms * 1e-3) / 1e12,
                         "hbm_frac": b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
                         "mfma_frac": f / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS}
    dominant = "gate_up" if ms_gu >= ms_dn else "down"
    k = kernels[dominant]
    # The metric's roofline: HBM bandwidth for decode-sized batches (the
    # weight-streaming kernels), MFMA peak for prefill; `binding_frac` is the
    # kernel's max(F / peak, B / BW) / t whichever binds.
    hbm_bound = layer.tile_rows <= 32
    t_floor = max(k["algorithmic_bytes"] / (HBM_PEAK_GBS * 1e9),
                  k["algorithmic_flops"] / (MFMA_BF16_PEAK_TFLOPS * 1e12))
    layout_name = "frag16" if layer.layout == tau.ffi.WEIGHTS_FRAG16 else "row_major"
    kernel_name = dominant + ("_fused" if layer.decode_path() else "")
    traffic = measured_traffic(shape.name, kernel_name, layout_name)
    ms_dom = k["us"] * 1e-3
    if hbm_bound:
        roofline = {"bound": "hbm", "achieved": k["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": k["hbm_frac"]}
    else:
        roofline = {"bound": "mfma", "achieved": k["TFLOP/s"], "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": k["mfma_frac"]}
    roofline.update({
        "traffic": traffic, "kernel": kernel_name,
        "kernel_symbol": ("decode_gemm_kernel" if layer.decode_path() else "mfma_gemm" if layer.tile_rows >= 64
                          else "stream_gemm_fast"),
        "kernel_us": k["us"],
        "binding_frac": t_floor / (k["us"] * 1e-6),
        "algorithmic_per_launch": {"bytes": k["algorithmic_bytes"], "flops": k["algorithmic_flops"]},
        # the same kernel against HBM, from its measured bytes (rocprofv3 FETCH/WRITE_SIZE)
        "traffic_GBs": traffic / ms_dom / 1e9 if traffic else None,
        "traffic_over_algorithmic": traffic / k["algorithmic_bytes"] if traffic else None,
        "kernels": kernels,
    })
    norm_report = None
    if layer.norm is not None:
        # algorithmic bytes: read x and branch, write residual and normalized (BF16), read the weight
        norm_bytes = 4 * T * H * 2 + H * 2
        layer.residual_norm()
        torch.cuda.synchronize()
        ms_norm = time_events(torch, layer.residual_norm, n_proj)
        norm_report = {"us": ms_norm * 1e3, "bytes": norm_bytes, "GB/s": norm_bytes / (ms_norm * 1e-3) / 1e9,
                       "hbm_frac": norm_bytes / (ms_norm * 1e-3) / 1e9 / HBM_PEAK_GBS}
    router_report = None
    if layer.router is not None:
        layer.route_from_hidden()
        layer.project_router()
        torch.cuda.synchronize()
        router_report = {"projection_and_routing_us": time_events(torch, layer.route_from_hidden, n_proj) * 1e3,
                         "projection_us": time_events(torch, layer.project_router, n_proj) * 1e3}
    layer_hbm = bytes_ / (ms_step * 1e-3) / 1e9
    layer_mfma = flops / (ms_step * 1e-3) / 1e12
    out = {
        "ms_per_step": ms_step,
        "tokens_per_s": T / (ms_step * 1e-3),
        "config": {
            "workload": shape.name, "tokens": T, "hidden": H, "experts": shape.experts, "top_k": K,
            "intermediate": I, "tile_rows": layer.tile_rows, "weight_banks": banks,
            "weight_layout": layout_name, "feed_forward_half": layer.norm is not None,
            "from_hidden_states": layer.router is not None,
            "shared_expert": ("folded" if layer.folded else "separate") if shape.shared_intermediate else None,
            "distinct_experts": distinct, "max_rows_per_expert": int(counts.max()), "plan_status": status,
        },
        "roofline": roofline,
        "layer_roofline": {
            "hbm_GBs": layer_hbm, "hbm_frac": layer_hbm / HBM_PEAK_GBS,
            "mfma_TFLOPs": layer_mfma, "mfma_frac": layer_mfma / MFMA_BF16_PEAK_TFLOPS,
            # max(F/peak, B/BW) / t: the fraction of the binding roofline
            "roofline_frac": max(flops / (MFMA_BF16_PEAK_TFLOPS * 1e12), bytes_ / (HBM_PEAK_GBS * 1e9))
                             / (ms_step * 1e-3),
            "algorithmic_bytes": bytes_, "algorithmic_flops": flops,
        },
        "timing": timing,
        "wall_s_timed": wall,
        **({"residual_norm": norm_report} if norm_report else {}),
        **({"router": router_report} if router_report else {}),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(layer, args.cpu_seconds)
    del layer
    torch.cuda.empty_cache()
    return out


def default_banks(shape, requested):
    weight_bytes = 3 * shape.hidden * shape.intermediate * 2 * shape.experts
    # 4 banks where they fit in 20 GB (every BASELINE layer does), far beyond the 256 MB MALL
    return requested or (4 if 4 * weight_bytes <= 2e10 else 2)


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every GPU box in this build has one MI355X and the MoE layer is "
              "benchmarked per GPU (expert-parallel sharding is a design note only); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    import torch

    if args.copy_calibration:
        copy_calibration(torch)
        return
    tau = load_package()
    shape = tau.inputs.CONFIGS[WORKLOADS[args.workload]]
    if args.tokens:
        shape = tau.inputs.scaled(shape, args.tokens)
    main_run = measure(tau, torch, shape, args, default_banks(shape, args.banks), args.steps, args.warmup,
                       args.workload)
    result = {
        "metric": "MoE-layer tokens/s; % bf16 MFMA peak (prefill), % HBM BW (decode)",
        "value": main_run["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_run["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) activations; random router)",
        **{k: v for k, v in main_run.items() if k not in ("tokens_per_s", "ms_per_step")},
    }
    # The prefill headline (c3: Qwen3-30B-A3B at 4096 tokens) in the same run
    # when the primary workload is the default decode one.
    if args.workload == "c2" and not args.tokens and not args.no_prefill:
        pshape = tau.inputs.CONFIGS[WORKLOADS["c3"]]
        pre = measure(tau, torch, pshape, args, default_banks(pshape, 0), args.steps, args.warmup, "c3 prefill")
        result["prefill"] = {"value": pre["tokens_per_s"], "unit": "tokens/s", "steps": args.steps,
                             "warmup": args.warmup, **{k: v for k, v in pre.items() if k != "tokens_per_s"}}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
