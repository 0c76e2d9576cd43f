#!/usr/bin/env python
"""Benchmark of the MI355X GPTQ-int4 W4A16 fused-MoE path.

Workload (one "step"): the decode sweep - 40 independent synthetic Qwen3.6-35B-A3B-shaped int4
MoE layers (hidden 2048, 256 experts, intermediate 512, top-8, group 128; router logits skewed to
Zipf(1.1) per layer), each layer = router -> align -> W1 -> W2 -> sum, captured as one hipGraph
chain per batch size and replayed at token batches 1, 8, 32 and 64. All weights (16.7 GB) are
resident in HBM before timing; the chain is larger than the 256 MB Infinity Cache, so every
expert read comes from HBM.

value = decode expert-weight HBM GB/s over the whole sweep: sum over batches and layers of
U_l(T) * 1 634 304 B (distinct routed experts x packed qweight+scales+qzeros per expert) divided
by the summed median chain time. Also reported: per-batch us/layer and GB/s, prefill-2048
TFLOP/s (103.08 GFLOP per layer) and the same layers at further batch sizes (256 and 8192 tokens
by default, on AUTO's path), the W1 decode kernel's roofline (live HIP events), and the CPU
baseline (the oracle's reference-faithful bf16 path on host cores, bounded sample).
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
sys.path.insert(0, str(ROOT))

METRIC = "int4 MoE-layer decode µs & HBM GB/s (bs 1–64); prefill-2048 TFLOP/s"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--layers", type=int, default=40)
    p.add_argument("--batches", default="1,8,32,64")
    p.add_argument("--prefill-tokens", type=int, default=2048)
    p.add_argument("--prefill-sizes", default="256,8192",
                   help="further token counts timed like the prefill batch (empty disables)")
    p.add_argument("--prefill-layers", type=int, default=8,
                   help="resident layers chained in the prefill graph (per-layer time: replay / "
                        "layers)")
    p.add_argument("--cpu-baseline-seconds", type=float, default=12.0,
                   help="wall-clock budget of the CPU baseline sample (0 disables it)")
    p.add_argument("--block-batches", default="1,32",
                   help="full-block batches (routed experts + gated int4 shared expert); empty disables")
    p.add_argument("--chain-batches", default="1,64",
                   help="decode-chain batches: the layers in a decode loop, each input the residual "
                        "stream's RMSNorm after the previous layer (empty disables)")
    p.add_argument("--offload-tokens", type=int, default=512,
                   help="decode steps of the offloaded-expert run at batch 1 (0 disables it)")
    p.add_argument("--offload-warmup", type=int, default=16)
    p.add_argument("--offload-slots", type=int, default=64, help="HBM slots per layer")
    p.add_argument("--prefetch-k", type=int, default=16, help="predicted experts prefetched per layer")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="first run a plain streaming kernel (fp32 negate) over this many MiB, three "
                        "times: the known-size dispatch that scales rocprofv3 FETCH_SIZE/WRITE_SIZE")
    p.add_argument("--json-out", default=None, help="also write the full result JSON here")
    return p.parse_args()


TRAFFIC_PROFILE = ROOT / "profiles" / "gemm_decode_w1_bs64_hbm_traffic.md"
# the sources of the W1 decode kernel whose digest the traffic summary records
TRAFFIC_SOURCES = ("mtp_amd/csrc/gemm_decode.hip", "mtp_amd/csrc/common.h")


def kernel_source_digest() -> str:
    import hashlib
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        h.update((ROOT / rel).read_bytes())
    return h.hexdigest()


def profiled_traffic(batch: int) -> tuple[float | None, str | None]:
    """HBM bytes per W1 decode launch at batch 64 from the committed rocprofv3 PMC summary
    (FETCH_SIZE and WRITE_SIZE scaled by a known-size streaming kernel), and why it is absent:
    None when the run measures another batch, the summary is missing, or the summary was
    collected on other kernel sources (its source digest differs from this tree's)."""
    if batch != 64:
        return None, "the summary covers batch 64"
    if not TRAFFIC_PROFILE.exists():
        return None, "no traffic summary"
    fields = {}
    for line in TRAFFIC_PROFILE.read_text().splitlines():
        for key in ("traffic_bytes_per_launch:", "kernel_sources_sha256:"):
            if line.startswith(key):
                fields[key] = line.split(":", 1)[1].strip()
    if fields.get("kernel_sources_sha256:") != kernel_source_digest():
        return None, "the summary was collected on other kernel sources"
    return float(fields["traffic_bytes_per_launch:"]), None


def median_event_ms(fn, steps: int, stream) -> list[float]:
    import torch
    times = []
    for _ in range(steps):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        times.append((a, b))
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in times]


def pct(xs: list[float], q: float) -> float:
    s = sorted(xs)
    return s[min(len(s) - 1, int(round(q * (len(s) - 1))))]


def main() -> int:
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the W4A16 MoE path runs on a "
                                   "single MI355X (expert-parallel sharding is design-only); "
                                   "run with --gpus 1"}))
        return 2

    import torch

    from mtp_amd import _lib, ops, synth

    _lib.load()  # fail loudly if the HIP library is missing
    torch.cuda.set_device(0)
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    batches = [int(b) for b in args.batches.split(",") if b]
    L = args.layers
    H, E, I, K = synth.HIDDEN, synth.NUM_EXPERTS, synth.INTERMEDIATE, synth.TOP_K
    per_expert = synth.expert_bytes()
    w1_per_expert = 2 * ((H // 8) * I * 4 + (H // 128) * I * 2 + (H // 128) * (I // 8) * 4)

    t0 = time.time()
    layers = [synth.make_layer(l, zipf=True, device=dev) for l in range(L)]
    torch.cuda.synchronize()
    resident = sum(ly.experts.nbytes_per_expert() * E for ly in layers)
    log(f"[bench] {L} layers resident: {resident / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    # The offload pools are allocated at start-up, as a server sizes its expert cache before
    # serving: allocated after the other sections' buffers, the HBM slot pool measured a lower
    # host->HBM copy rate (perfect-predictor TPOT 3.38 vs 2.81 ms on one box).
    offload_pool = make_offload_pool(layers, args, dev) if args.offload_tokens > 0 else None

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log(f"[bench] calibration: 3 x negate of {args.copy_calibration_mib} MiB (reads and writes "
            f"{n * 4} B each)")
        del src, dst

    # ------------------------------------------------------------------ decode sweep
    graphs, decode = {}, {}
    keep = []
    for T in batches:
        x = synth.make_tokens(T, seed=7, device=dev)
        need = ops.workspace_bytes(T, K, layers[0].experts, False, "decode")
        ws = torch.zeros(need, dtype=torch.uint8, device=dev)
        outs = [torch.empty(T, H, dtype=torch.bfloat16, device=dev) for _ in range(L)]
        uniq = []
        for l, ly in enumerate(layers):
            _, ids, _ = ops.moe_layer(x, ly.router_w, ly.experts, top_k=K, logit_bias=ly.logit_bias,
                                      workspace=ws, out=outs[l], return_routing=True,
                                      path="decode")
            uniq.append(int(torch.unique(ids).numel()))
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for l, ly in enumerate(layers):
                ops.moe_layer(x, ly.router_w, ly.experts, top_k=K, logit_bias=ly.logit_bias,
                              workspace=ws, out=outs[l], path="decode")
        graphs[T] = g
        keep.append((x, ws, outs))
        decode[T] = {"U_per_layer_mean": sum(uniq) / L, "bytes": sum(uniq) * per_expert}
        log(f"[bench] captured bs={T}: mean distinct experts/layer {sum(uniq) / L:.1f}")

    for _ in range(args.warmup):
        for T in batches:
            graphs[T].replay()
    torch.cuda.synchronize()
    per_batch_times = {T: [] for T in batches}
    ev = []
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    for _ in range(args.steps):
        for T in batches:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            graphs[T].replay()
            b.record(stream)
            ev.append((T, a, b))
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    for T, a, b in ev:
        per_batch_times[T].append(a.elapsed_time(b))
    total_bytes = total_ms = 0.0
    for T in batches:
        ts = per_batch_times[T]
        med = statistics.median(ts)
        d = decode[T]
        d.update({
            "chain_ms_p50": med,
            "us_per_layer_p50": med * 1e3 / L,
            "us_per_layer_p95": pct(ts, 0.95) * 1e3 / L,
            "GBps": d["bytes"] / (med * 1e-3) / 1e9,
        })
        d["hbm_frac"] = d["GBps"] / HBM_PEAK_GBPS
        total_bytes += d["bytes"]
        total_ms += med
        log(f"[bench] decode bs={T}: {d['us_per_layer_p50']:.2f} us/layer, {d['GBps']:.0f} GB/s "
            f"({100 * d['hbm_frac']:.1f}% of 8 TB/s), U={d['U_per_layer_mean']:.1f}")
    agg_gbps = total_bytes / (total_ms * 1e-3) / 1e9

    # ------------------------------------------------------ dominant kernel: W1 decode at bs=64
    Tr = max(batches)
    x = keep[batches.index(Tr)][0]
    routed = []
    for ly in layers:
        ids, w, _, _ = ops.router_topk(x, ly.router_w, K, logit_bias=ly.logit_bias)
        s, e, n = ops.align(ids, E, ops.DECODE_BLOCK_M)
        routed.append((s, e, n, int(torch.unique(ids).numel())))
    hbuf = torch.empty(Tr * K, I, dtype=torch.bfloat16, device=dev)
    structs = [ly.experts.struct() for ly in layers]
    lib = _lib.load()
    import ctypes

    def w1_chain():
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for ly, ex, (s, e, n, _) in zip(layers, structs, routed):
            _lib.check(lib.moe_w1_gateup_silu_v1(x.data_ptr(), Tr, K, ctypes.byref(ex), None,
                                                 s.data_ptr(), e.data_ptr(), n.data_ptr(),
                                                 ops.DECODE_BLOCK_M, e.numel(), hbuf.data_ptr(),
                                                 ops.PATHS["decode"], st))
    w1_chain()
    torch.cuda.synchronize()
    gw1 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gw1):
        w1_chain()
    for _ in range(args.warmup):
        gw1.replay()
    w1_ms = statistics.median(median_event_ms(gw1.replay, args.steps, stream))
    w1_launch_us = w1_ms * 1e3 / L
    w1_bytes_per_launch = sum(r[3] for r in routed) * w1_per_expert / L
    traffic, traffic_note = profiled_traffic(Tr)
    roofline = {
        "bound": "hbm",
        "kernel": f"gemm_decode_kernel<W1> (gate_up + SiLU*mul), bs={Tr}",
        "achieved": w1_bytes_per_launch / (w1_launch_us * 1e-6) / 1e9,
        "peak": HBM_PEAK_GBPS,
        "unit": "GB/s",
        "traffic": traffic,
        "traffic_source": (f"{TRAFFIC_PROFILE.name} (kernel sources sha256 "
                           f"{kernel_source_digest()[:12]})") if traffic else traffic_note,
        "launch_us": w1_launch_us,
        "algorithmic_bytes_per_launch": w1_bytes_per_launch,
    }
    roofline["frac"] = roofline["achieved"] / roofline["peak"]
    log(f"[bench] W1 decode bs={Tr}: {w1_launch_us:.2f} us/launch, {roofline['achieved']:.0f} GB/s")

    # ------------------------------- W1 / W2 latency buckets (the reference's measurement unit)
    # W1 = gate_up of 1 token x top-8, W2 = down of those 8 rows with top_k = 1, each launch
    # bracketed by its own HIP events (eager, not captured), as the reference's GPU-event
    # latencies of the wna16 kernels (vllm_router_trace.py:14321-14326, reduced to p50/p95/p99
    # by summarize_wna16_w1w2_timing.py:13-28).
    buckets = {}
    if True:
        xb = synth.make_tokens(1, seed=7, device=dev)
        hb = torch.empty(K, I, dtype=torch.bfloat16, device=dev)
        yb = torch.empty(K, H, dtype=torch.float32, device=dev)
        routed1 = []
        for ly in layers:
            ids1, w1_, _, _ = ops.router_topk(xb, ly.router_w, K, logit_bias=ly.logit_bias)
            s1, e1, n1 = ops.align(ids1, E, ops.DECODE_BLOCK_M)
            routed1.append((s1, e1, n1, w1_.reshape(-1).contiguous()))
        st1 = ctypes.c_void_p(stream.cuda_stream)

        def w1_launch(ex, r):
            _lib.check(lib.moe_w1_gateup_silu_v1(xb.data_ptr(), 1, K, ctypes.byref(ex), None,
                                                 r[0].data_ptr(), r[1].data_ptr(), r[2].data_ptr(),
                                                 ops.DECODE_BLOCK_M, r[1].numel(), hb.data_ptr(),
                                                 ops.PATHS["decode"], st1))

        def w2_launch(ex, r):
            _lib.check(lib.moe_w2_down_v1(hb.data_ptr(), 1, K, ctypes.byref(ex), None,
                                          r[0].data_ptr(), r[1].data_ptr(), r[2].data_ptr(),
                                          ops.DECODE_BLOCK_M, r[1].numel(), r[3].data_ptr(),
                                          yb.data_ptr(), ops.PATHS["decode"], st1))
        samples = {"w1": [], "w2": []}
        for rep in range(args.warmup + max(args.steps // 2, 5)):
            evs = []
            for ex, r in zip(structs, routed1):
                for name, fn in (("w1", w1_launch), ("w2", w2_launch)):
                    a = torch.cuda.Event(enable_timing=True)
                    b = torch.cuda.Event(enable_timing=True)
                    a.record(stream)
                    fn(ex, r)
                    b.record(stream)
                    evs.append((name, a, b))
            torch.cuda.synchronize()
            if rep >= args.warmup:
                for name, a, b in evs:
                    samples[name].append(a.elapsed_time(b) * 1e3)
        for name, xs in samples.items():
            buckets[name + "_us"] = {"p50": pct(xs, 0.5), "p95": pct(xs, 0.95), "p99": pct(xs, 0.99),
                                     "samples": len(xs)}
        buckets["workload"] = (f"batch 1 over the {L} Zipf layers: W1 = gate_up + SiLU*mul of 1 token "
                               f"x top-{K} (moe_w1_gateup_silu_v1), W2 = down of those {K} rows with "
                               "top_k = 1 and the routed weight (moe_w2_down_v1); one HIP event pair "
                               "per eager launch")
        buckets["reference_w7900"] = {"w1_us": {"p50": 135.05, "p95": 148.63},
                                      "w2_us": {"p50": 79.71, "p95": 96.45},
                                      "source": "PROGRESS.md:19498-19509 (vLLM Triton wna16, AWQ, "
                                                "Radeon PRO W7900)"}
        log(f"[bench] W1/W2 buckets bs=1: W1 p50 {buckets['w1_us']['p50']:.2f} us "
            f"p95 {buckets['w1_us']['p95']:.2f}; W2 p50 {buckets['w2_us']['p50']:.2f} us "
            f"p95 {buckets['w2_us']['p95']:.2f}")

    # ------------------------------------------------------------------ prefill-2048
    # A chain of the first `prefill_layers` resident layers in one graph (as the decode chains),
    # per-layer time = replay / layers; layer 0 alone per replay is reported beside it.
    def measure_prefill(Tp: int, NLp: int) -> dict:
        xp = synth.make_tokens(Tp, seed=7, device=dev)
        wsps, outps, us = [], [], []
        counts = None
        for ly in layers[:NLp]:
            need = ops.workspace_bytes(Tp, K, ly.experts, False, "auto")
            wsps.append(torch.zeros(need, dtype=torch.uint8, device=dev))
            outps.append(torch.empty(Tp, H, dtype=torch.bfloat16, device=dev))
            _, ids, _ = ops.moe_layer(xp, ly.router_w, ly.experts, top_k=K,
                                      logit_bias=ly.logit_bias, workspace=wsps[-1],
                                      out=outps[-1], return_routing=True)
            c = torch.bincount(ids.view(-1).long(), minlength=E)
            counts = c if counts is None else counts
            us.append(int((c > 0).sum()))

        def prefill_chain(n):
            for i in range(n):
                ly = layers[i]
                ops.moe_layer(xp, ly.router_w, ly.experts, top_k=K, logit_bias=ly.logit_bias,
                              workspace=wsps[i], out=outps[i])

        def replay_ms(n):
            gp = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gp):
                prefill_chain(n)
            for _ in range(args.warmup):
                gp.replay()
            return statistics.median(median_event_ms(gp.replay, args.steps, stream)) / n

        med = replay_ms(NLp)
        single = replay_ms(1) if NLp > 1 else med
        flops = synth.prefill_flops(Tp)
        prefill = {
            "tokens": Tp,
            "layers_in_chain": NLp,
            "layer_us_p50": med * 1e3,
            "single_layer_us_p50": single * 1e3,
            "TFLOPs": flops / (med * 1e-3) / 1e12,
            "flop": flops,
            "expert_tokens_max": int(counts.max()),
            "expert_tokens_min": int(counts.min()),
            "experts_with_zero_tokens": int((counts == 0).sum()),
        }
        prefill["mfma_frac"] = prefill["TFLOPs"] / MFMA_BF16_PEAK_TFLOPS
        # HBM co-bound: the routed experts' bytes (each read at least once) over the same time;
        # the router's FLOPs are reported apart from the useful expert FLOPs
        prefill["expert_bytes"] = statistics.mean(us) * synth.expert_bytes()
        prefill["GBps"] = prefill["expert_bytes"] / (med * 1e-3) / 1e9
        prefill["hbm_frac"] = prefill["GBps"] / HBM_PEAK_GBPS
        prefill["router_flop"] = 2 * Tp * E * H
        prefill["path"] = "prefill" if Tp * K >= ops.AUTO_PREFILL_SLOTS else "decode"
        log(f"[bench] prefill T={Tp}: {med * 1e3:.1f} us/layer over {NLp} chained layers "
            f"(layer 0 alone per replay {single * 1e3:.1f} us), {prefill['TFLOPs']:.1f} TFLOP/s "
            f"({100 * prefill['mfma_frac']:.1f}% of bf16 MFMA peak); expert bytes "
            f"{prefill['expert_bytes'] / 1e6:.1f} MB at {prefill['GBps']:.0f} GB/s "
            f"({100 * prefill['hbm_frac']:.1f}% of 8 TB/s); {prefill['path']} kernels")
        return prefill

    NLp = max(1, min(args.prefill_layers, len(layers)))
    prefill = measure_prefill(args.prefill_tokens, NLp) if args.prefill_tokens > 0 else {}
    # other batch sizes through the same layers (AUTO's path), reported beside the headline
    prefill_sizes = [measure_prefill(t, NLp) for t in
                     (int(v) for v in args.prefill_sizes.split(",") if v) if t > 0]

    # ------------------------------------------------------- full block with shared expert
    block = {}
    block_batches = [int(b) for b in args.block_batches.split(",") if b]
    if block_batches:
        from mtp_amd.weights import MoeExperts  # noqa: F401  (shared experts are MoeExperts)
        shared = [synth.make_experts(1, H, I, seed=4000 + l, device=dev) for l in range(L)]
        sgate = [synth.make_shared_gate(H, seed=2500 + l, device=dev) for l in range(L)]
        for T in block_batches:
            x = synth.make_tokens(T, seed=7, device=dev)
            need = ops.workspace_bytes(T, K, layers[0].experts, True, "auto")
            ws = torch.zeros(need, dtype=torch.uint8, device=dev)
            outs = [torch.empty(T, H, dtype=torch.bfloat16, device=dev) for _ in range(L)]
            uniq = []
            for l, ly in enumerate(layers):
                _, ids, _ = ops.moe_layer(x, ly.router_w, ly.experts, top_k=K, logit_bias=ly.logit_bias,
                                          shared=shared[l], shared_gate_w=sgate[l], workspace=ws,
                                          out=outs[l], return_routing=True)
                uniq.append(int(torch.unique(ids).numel()))
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for l, ly in enumerate(layers):
                    ops.moe_layer(x, ly.router_w, ly.experts, top_k=K, logit_bias=ly.logit_bias,
                                  shared=shared[l], shared_gate_w=sgate[l], workspace=ws, out=outs[l])
            for _ in range(args.warmup):
                g.replay()
            ts = median_event_ms(g.replay, args.steps, stream)
            med = statistics.median(ts)
            nbytes = (sum(uniq) + L) * per_expert
            block[str(T)] = {"us_per_layer_p50": med * 1e3 / L, "us_per_layer_p95": pct(ts, 0.95) * 1e3 / L,
                             "GBps": nbytes / (med * 1e-3) / 1e9,
                             "U_per_layer_mean": sum(uniq) / L, "shared_experts_per_layer": 1}
            log(f"[bench] block bs={T}: {block[str(T)]['us_per_layer_p50']:.2f} us/layer "
                f"{block[str(T)]['GBps']:.0f} GB/s (routed + shared expert bytes)")
            del g, ws, outs
        del shared, sgate

    # ------------------------------------- decode chain: the layers in a decode loop (dependent)
    # Per layer l: res = res + y_{l-1}; h = RMSNorm_l(res); y_l = MoE_l(h) (the decoder loop around
    # moe_forward_with_trace with mtp_rms_norm), then the final RMSNorm_L, so every layer's routing
    # depends on the previous layer's output. Each step of the timed loop is one
    # moe_norm_layer_v1 call (the router normalises its own tokens) on two alternating residual
    # buffers; the bits equal the rmsnorm + moe_layer loop, which records the routing. Same
    # layers, weights and routing bias as the sweep.
    chain = {}
    chain_batches = [int(b) for b in args.chain_batches.split(",") if b]
    if chain_batches:
        gn = torch.Generator().manual_seed(6000)
        norm_w = [(0.05 * torch.randn(H, generator=gn)).to(torch.bfloat16).to(dev) for _ in range(L + 1)]
        for T in chain_batches:
            x0 = synth.make_tokens(T, seed=7, device=dev)
            res = torch.empty_like(x0)
            h = torch.empty_like(x0)
            y = torch.empty_like(x0)
            ws = torch.zeros(ops.workspace_bytes(T, K, layers[0].experts, False, "decode"),
                             dtype=torch.uint8, device=dev)

            res2 = torch.empty_like(x0)

            def record_routing(record):
                res.copy_(x0)
                ops.rmsnorm(res, norm_w[0], out=h)
                for l, ly in enumerate(layers):
                    _, ids, _ = ops.moe_layer(h, ly.router_w, ly.experts, top_k=K,
                                              logit_bias=ly.logit_bias, workspace=ws, out=y,
                                              return_routing=True, path="decode")
                    record.append(int(torch.unique(ids).numel()))
                    ops.rmsnorm(res, norm_w[l + 1], add=y, out=h)

            def chain_step():
                bufs = (res, res2)
                res.copy_(x0)
                cur = 0
                for l, ly in enumerate(layers):
                    ops.norm_layer(bufs[cur], ly.router_w, ly.experts, norm_w[l],
                                   add=y if l else None, res_out=bufs[1 - cur], x_out=h, top_k=K,
                                   logit_bias=ly.logit_bias, workspace=ws, out=y, path="decode")
                    cur = 1 - cur
                ops.rmsnorm(bufs[cur], norm_w[L], add=y, out=h)

            uniq = []
            record_routing(uniq)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                chain_step()
            for _ in range(args.warmup):
                g.replay()
            ts = median_event_ms(g.replay, args.steps, stream)
            med = statistics.median(ts)
            nbytes = sum(uniq) * per_expert
            chain[str(T)] = {"tpot_ms_p50": med, "us_per_layer_p50": med * 1e3 / L,
                             "us_per_layer_p95": pct(ts, 0.95) * 1e3 / L,
                             "GBps": nbytes / (med * 1e-3) / 1e9, "U_per_layer_mean": sum(uniq) / L}
            log(f"[bench] decode chain bs={T}: {med:.3f} ms per step ({L} layers + norms), "
                f"{chain[str(T)]['us_per_layer_p50']:.2f} us/layer, {chain[str(T)]['GBps']:.0f} GB/s, "
                f"U={sum(uniq) / L:.1f}")
            del g, ws

    # ------------------------------------------------------------------ offloaded experts
    offload = None
    if args.offload_tokens > 0:
        del graphs, keep, gw1
        torch.cuda.synchronize()
        offload = offload_bench(layers, offload_pool, args, dev)
        offload_pool = None

    # ------------------------------------------------------------------ CPU baseline
    cpu = None
    if args.cpu_baseline_seconds > 0:
        cpu = cpu_baseline(layers, batches, args.cpu_baseline_seconds, per_expert,
                           max(args.prefill_tokens, 0), block_batches)

    result = {
        "metric": METRIC,
        "value": agg_gbps,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded random int4 GPTQ weights, N(0,1) bf16 tokens, Zipf(1.1)-skewed router)",
        "config": {
            "workload": f"decode sweep: {L} independent int4 MoE layers (H{H} E{E} I{I} top-{K}, group 128), "
                        f"one hipGraph chain per batch, batches {batches}; value = expert-weight HBM GB/s "
                        "over the sweep",
            "layers": L, "batches": batches, "hidden": H, "experts": E, "intermediate": I,
            "top_k": K, "group_size": 128, "weights_resident_GB": resident / 1e9,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "decode": {str(T): decode[T] for T in batches},
        "decode_buckets": buckets,
        "prefill": prefill,
        "prefill_sizes": prefill_sizes,
        "block": block,
        "decode_chain": chain,
        "offload": offload,
    }
    line = json.dumps(result)
    if args.json_out:
        Path(args.json_out).write_text(json.dumps(result, indent=2))
    print(line, flush=True)
    return 0


def make_offload_pool(layers, args, dev):
    """Pinned host pool of every (layer, expert) blob and the HBM slot pool, filled."""
    import torch

    from mtp_amd import synth
    from mtp_amd.offload import OffloadedExperts

    t0 = time.time()
    pool = OffloadedExperts(len(layers), synth.NUM_EXPERTS, synth.HIDDEN, synth.INTERMEDIATE,
                            args.offload_slots, device=dev)
    for l, ly in enumerate(layers):
        pool.store_layer(l, ly.experts)
    torch.cuda.synchronize()
    log(f"[bench] offload: host pool {pool.host.nbytes / 1e9:.2f} GB pinned, HBM pool "
        f"{pool.device_pool.numel() / 1e9:.2f} GB, filled in {time.time() - t0:.1f}s")
    return pool


def offload_bench(layers, pool, args, dev) -> dict:
    """Offloaded experts at batch 1: every (layer, expert) blob in pinned host memory, an HBM pool
    of `offload_slots` slots per layer, per-layer predictor heads (bf16 2048 -> 1024 SiLU -> 256,
    random init) reading h = 0.8 x_next + 0.6 eps, top-`prefetch_k` prefetched on the side stream,
    misses fetched on demand. Four runs over the same token sequence: the random-init MLP
    predictor, a random-init HiddenResidualExpertPredictor (the reference's predictor
    architecture), no prefetch (demand only) and a perfect predictor (the next step's true routed
    experts)."""
    import torch

    from mtp_amd import ops, synth
    from mtp_amd.offload import OffloadDecoder

    L, E, H, K = len(layers), synth.NUM_EXPERTS, synth.HIDDEN, synth.TOP_K
    D = 1024
    n_tok = args.offload_warmup + args.offload_tokens
    calib = h2d_calibration(pool)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5000)
    w1 = (torch.randn(L, D, H, generator=gen, device=dev) / H ** 0.5).to(torch.bfloat16)
    w2 = (torch.randn(L, E, D, generator=gen, device=dev) / D ** 0.5).to(torch.bfloat16)
    xs = torch.randn(n_tok + 1, 1, H, generator=gen, device=dev).to(torch.bfloat16)
    eps = torch.randn(n_tok + 1, 1, H, generator=gen, device=dev)
    hs = (0.8 * xs.float() + 0.6 * eps).to(torch.bfloat16)
    routers = [ly.router_w for ly in layers]
    biases = [ly.logit_bias for ly in layers]
    # true routed experts of every step (for the perfect-predictor run)
    true_ids = []
    for t in range(n_tok + 1):
        per_layer = []
        for ly in layers:
            ids, _, _, _ = ops.router_topk(xs[t], ly.router_w, K, logit_bias=ly.logit_bias)
            per_layer.append(ids)
        true_ids.append(torch.stack(per_layer))
    true_host = torch.stack(true_ids).cpu()
    true_lists = [[list(dict.fromkeys(true_host[t, l].reshape(-1).tolist())) for l in range(L)]
                  for t in range(n_tok + 1)]

    from mtp_amd.predictor import HiddenResidualExpertPredictor
    hr = HiddenResidualExpertPredictor(hidden_size=H, num_experts=E, num_layers=L, seed=5001,
                                       device=dev)
    runs = {}
    for name, predictor, k in (("random_predictor", (w1, w2), args.prefetch_k),
                               ("hidden_residual_predictor", hr, args.prefetch_k),
                               ("demand_only", None, 0),
                               ("perfect_predictor", None, K)):
        pool.reset_cache()
        fresh = pool
        dec = OffloadDecoder(fresh, routers, biases, top_k=K, predictor=predictor, prefetch_k=k,
                             path="decode")
        step_s, base, trace = [], None, []
        for t in range(n_tok):
            if t == args.offload_warmup:
                torch.cuda.synchronize()
                base = fresh.stats()
            t1 = time.perf_counter()
            if name == "perfect_predictor":
                pre = true_lists[t + 1]
            else:
                pre = dec.predict(hs[t + 1])
            outs = dec.step(xs[t], pre, trace=trace)
            torch.cuda.current_stream().synchronize()
            if t >= args.offload_warmup:
                step_s.append(time.perf_counter() - t1)
        # spot check of the last step (outside the timing): every layer's output read from the
        # slots equals the resident layer's, bit for bit
        spot = all(torch.equal(outs[l], ops.moe_layer(xs[n_tok - 1], ly.router_w, ly.experts,
                                                      top_k=K, logit_bias=ly.logit_bias,
                                                      path="decode"))
                   for l, ly in enumerate(layers))
        torch.cuda.synchronize()
        st = fresh.stats()
        diff = {k2: st[k2] - base[k2] for k2 in st if k2 not in ("capacity", "resident_count",
                                                                  "unused_fetch_count")}
        diff["unused_fetch_count"] = st["unused_fetch_count"]
        total = sum(step_s)
        runs[name] = {
            "tpot_ms_mean": 1e3 * total / len(step_s),
            "tpot_ms_p50": 1e3 * statistics.median(step_s),
            "tpot_ms_p95": 1e3 * pct(step_s, 0.95),
            "hit_rate": diff["demand_hit_count"] / max(diff["demand_count"], 1),
            # the reference's ready-time semantics count a hit whose copy arrived late as a miss
            "ready_hit_rate": (diff["demand_hit_count"] - diff["ready_late_miss_count"])
                              / max(diff["demand_count"], 1),
            "h2d_GBps": (diff["prefetch_bytes"] + diff["demand_bytes"]) / total / 1e9,
            "counters": diff,
            "last_step_equals_resident_layers": bool(spot),
            "reference_semantics": ready_time_replay(trace, L * args.offload_slots,
                                                     calib["two_streams_us_per_expert"]["p50"],
                                                     args.offload_warmup * L),
        }
        rs = runs[name]["reference_semantics"]
        log(f"[bench] offload {name}: TPOT {runs[name]['tpot_ms_mean']:.2f} ms, hit rate "
            f"{100 * runs[name]['hit_rate']:.1f}% (ready in time {100 * runs[name]['ready_hit_rate']:.1f}%, "
            f"{diff['ready_late_miss_count']} ready-late), H2D {runs[name]['h2d_GBps']:.1f} GB/s; "
            f"ReadyTimeExpertCacheManager replay: hit rate {100 * rs['hit_rate']:.1f}%, "
            f"{rs['ready_late_miss_count']} ready-late misses")
    pool.close()
    del pool
    return {
        "workload": f"batch 1, {args.offload_tokens} decode steps after {args.offload_warmup} warmup, "
                    f"{L} layers x {E} experts in pinned host memory, {args.offload_slots} HBM slots/layer, "
                    f"prefetch top-{args.prefetch_k} per layer of a random-init bf16 predictor (per-layer "
                    "2048 -> 1024 SiLU -> 256 heads) or of a random-init HiddenResidualExpertPredictor "
                    "(width 256, 4 future deltas; delta 0 used); ready-late = first demand of a "
                    "prefetched expert whose copy completed after the demand (HIP event times)",
        "runs": runs,
        "h2d_calibration": calib,
    }


def ready_time_replay(trace, capacity: int, service_us: float, skip: int) -> dict:
    """The offload run's call sequence (per layer call: demanded ids, then the prefetch list, at
    the host time the call made them) through the reference's ReadyTimeExpertCacheManager
    (cache_manager.py:298-578, native): one LRU of `capacity` keys, each issue a transfer of
    `service_us` (the measured pinned H2D time per expert when copies alternate over two
    streams, as the slot cache's prefetches do), batches of one, no deadline. A
    demand then hits only experts whose virtual transfer completed by its arrival; a demand of
    one still in flight is a ready-late miss. Counters cover the calls after the first `skip`
    (the warmup steps), as the measured counters do."""
    from mtp_amd.cache_manager import ReadyTimeExpertCacheManager
    m = ReadyTimeExpertCacheManager(capacity=capacity, service_us_per_issue=service_us)
    t0 = trace[0][3] if trace else 0.0
    base = None
    for i, (layer, ids, pre, t_us) in enumerate(trace):
        if i == skip:
            base = m.snapshot().as_dict()
        m.demand_many(layer, ids, arrival_us=t_us - t0)
        m.issue_prefetches(layer, pre, arrival_us=t_us - t0)
    m.finish()
    s = m.snapshot().as_dict()
    base = base or {k: 0 for k in s}
    keys = ("issued_fetch_count", "used_fetch_count", "demand_count", "demand_hit_count",
            "demand_miss_count", "evicted_before_use_count", "ready_late_miss_count",
            "late_completion_unused_count")
    d = {k: int(s[k] - base[k]) for k in keys}
    d["hit_rate"] = d["demand_hit_count"] / max(d["demand_count"], 1)
    d.update({"capacity": capacity, "service_us_per_issue": service_us,
              "arrival": "host time of each layer call (demand, then the prefetch list)"})
    return d


def h2d_calibration(pool, reps: int = 200) -> dict:
    """Pinned host -> HBM copy of expert blobs with hipMemcpyAsync (the slot cache's copy), timed
    with HIP events on one stream: single blobs and batches of 8, p50 / p95, beside the reference's
    measured copy (W7900, PCIe 4.0 x16); then batches of 16 split over two streams, as the slot
    cache's two copy streams move prefetches (the per-expert service time of its transfers)."""
    import ctypes

    import torch

    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpyAsync.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                   ctypes.c_void_p]
    hip.hipMemcpyAsync.restype = ctypes.c_int
    blob, n_blobs = pool.blob, pool.num_layers * pool.num_experts
    dst = pool.device_pool.view(-1)
    n_dst = dst.numel() // blob
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    def copy(i: int) -> None:
        src = pool.host.ptr + (i * 7919 % n_blobs) * blob  # blobs spread over the pool
        err = hip.hipMemcpyAsync(ctypes.c_void_p(dst.data_ptr() + (i % n_dst) * blob),
                                 ctypes.c_void_p(src), blob, 1, sh)  # 1 = host to device
        if err != 0:
            raise RuntimeError(f"hipMemcpyAsync failed with HIP error {err}")

    def timed(n: int, rep: int) -> float:
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for j in range(n):
            copy(rep * n + j)
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) * 1e3  # us

    side = [torch.cuda.Stream(), torch.cuda.Stream()]

    def timed_two(n: int, rep: int) -> float:  # n blobs alternating over the two side streams
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for st in side:
            st.wait_stream(stream)
        for j in range(n):
            i = rep * n + j
            src = pool.host.ptr + (i * 7919 % n_blobs) * blob
            err = hip.hipMemcpyAsync(ctypes.c_void_p(dst.data_ptr() + (i % n_dst) * blob),
                                     ctypes.c_void_p(src), blob, 1,
                                     ctypes.c_void_p(side[j % 2].cuda_stream))
            if err != 0:
                raise RuntimeError(f"hipMemcpyAsync failed with HIP error {err}")
        for st in side:
            stream.wait_stream(st)
        b.record(stream)
        b.synchronize()
        return a.elapsed_time(b) * 1e3  # us

    for r in range(10):
        timed(8, r)
        timed_two(16, r)
    one = [timed(1, r) for r in range(reps)]
    eight = [timed(8, r) for r in range(reps // 2)]
    two = [timed_two(16, r) for r in range(reps // 2)]
    out = {
        "expert_bytes": blob,
        "one_expert_us": {"p50": statistics.median(one), "p95": pct(one, 0.95)},
        "one_expert_GBps_p95": blob / pct(one, 0.95) / 1e3,
        "one_expert_GBps_p50": blob / statistics.median(one) / 1e3,
        "eight_experts_us_per_expert": {"p50": statistics.median(eight) / 8,
                                        "p95": pct(eight, 0.95) / 8},
        "eight_experts_GBps_p50": 8 * blob / statistics.median(eight) / 1e3,
        "two_streams_us_per_expert": {"p50": statistics.median(two) / 16,
                                      "p95": pct(two, 0.95) / 16},
        "two_streams_GBps_p50": 16 * blob / statistics.median(two) / 1e3,
        "samples": {"one": len(one), "eight": len(eight), "two_streams": len(two)},
        "reference_w7900_pcie4": {"one_expert_GBps_p95": 20.43, "eight_experts_GBps_p50": 28.23,
                                  "eight_experts_us_per_expert_p95": 62.09,
                                  "expert_bytes": 1.65e6,
                                  "source": "PROGRESS.md:48610-48612"},
    }
    log(f"[bench] H2D calibration: 1 expert ({blob / 1e6:.2f} MB) p50 {out['one_expert_us']['p50']:.1f} us "
        f"p95 {out['one_expert_us']['p95']:.1f} us ({out['one_expert_GBps_p95']:.1f} GB/s at p95); "
        f"8 experts {out['eight_experts_GBps_p50']:.1f} GB/s at p50, "
        f"{out['eight_experts_us_per_expert']['p95']:.1f} us per expert at p95; 16 experts over two "
        f"streams {out['two_streams_GBps_p50']:.1f} GB/s at p50")
    return out


CPU_REPS = 5


def _cpu_threads() -> tuple[int, int]:
    """(threads used, cores in this process's affinity set). The harness of a shared GPU box sets
    OMP_NUM_THREADS to the box's CPU share; the baseline then uses that share, else every core of
    the affinity set."""
    affinity = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS")
    threads = min(affinity, int(share)) if share and share.isdigit() and int(share) > 0 else affinity
    return threads, affinity


def _cpu_layer(ly, torch):
    return (ly.router_w.cpu(), ly.logit_bias.cpu() if ly.logit_bias is not None else None,
            {n: (st.qweight.cpu(), st.qzeros.cpu(), st.scales.cpu())
             for n, st in (("gate", ly.experts.gate), ("up", ly.experts.up), ("down", ly.experts.down))})


def _cpu_dequant(stacks, used, moe_ref, torch):
    sel = torch.tensor(used)
    deq = {n: torch.cat([moe_ref.dequant_stack_torch(q[c], z[c], s[c]) for c in sel.split(32)])
           for n, (q, z, s) in stacks.items()}
    return {e: (deq["gate"][i], deq["up"][i], deq["down"][i]) for i, e in enumerate(used)}


def _cpu_route(x, router, bias, F, torch):
    lg = F.linear(x, router).float()
    if bias is not None:
        lg = lg + bias
    p = torch.softmax(lg, dim=-1)
    w, ids = torch.topk(p, 8, dim=-1)
    return ids, w / w.sum(-1, keepdim=True).clamp_min(1e-20)


def cpu_baseline(layers, batches, budget_s: float, per_expert: int, prefill_tokens: int,
                 block_batches: list[int]) -> dict:
    """The oracle's reference-faithful CPU path timed on the host cores (not the optimisation
    target): dequantise at load (gptq_unpack.py:88-131), then per call the fp32 router
    (softmax -> top-8 -> renormalise) and the moe_tokens slot loop of bf16 F.linear per routed
    expert (extra_tensors.py:544-598). Median of CPU_REPS repetitions per case.
      * decode: layers 0..3 at every decode batch (a bounded sample of the 40-layer sweep; the
        GB/s figure uses the same algorithmic expert bytes as the GPU metric);
      * prefill: the full prefill batch through layer 0 (TFLOP/s on the same useful FLOPs);
      * full block: the decode block batches through layer 0 with a gated int4 shared expert.
    The dequant-inclusive variant adds the dequantisation of the routed experts to each call."""
    import torch
    import torch.nn.functional as F

    from mtp_amd import synth
    from oracle import moe_ref

    threads, affinity = _cpu_threads()
    torch.set_num_threads(threads)
    t_start = time.time()

    def timed(fn):
        reps = []
        for _ in range(CPU_REPS):
            t1 = time.perf_counter()
            fn()
            reps.append(time.perf_counter() - t1)
        return statistics.median(reps)

    sample_layers = min(4, len(layers))
    tot_bytes = tot_s = tot_s_deq = 0.0
    done = []
    for l in range(sample_layers):
        router, bias, stacks = _cpu_layer(layers[l], torch)
        for T in batches:
            if time.time() - t_start > budget_s:
                break
            x = synth.make_tokens(T, seed=7).to(torch.bfloat16)
            ids, _ = _cpu_route(x, router, bias, F, torch)
            used = torch.unique(ids).tolist()
            t_deq = time.perf_counter()
            experts = _cpu_dequant(stacks, used, moe_ref, torch)
            t_deq = time.perf_counter() - t_deq

            def call():
                ii, ww = _cpu_route(x, router, bias, F, torch)
                moe_ref.moe_tokens_bf16(x, ii, ww, experts)
            med = timed(call)
            tot_bytes += len(used) * per_expert
            tot_s += med
            tot_s_deq += med + t_deq
            done.append(f"L{l}/bs{T}")
    if tot_s == 0:
        return None
    out = {
        "value": tot_bytes / tot_s / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "affinity_cores": affinity,
        "kind": "port",
        "sample": f"reference-faithful bf16 path (dequantise at load, bf16 F.linear per routed expert, "
                  f"moe_tokens slot loop) on layers x batches {done}, median of {CPU_REPS} reps "
                  "each; same algorithmic expert bytes as the GPU metric",
        "dequant_inclusive_GBps": tot_bytes / tot_s_deq / 1e9,
        "torch": torch.__version__,
        "cpu_model": _cpu_model(),
    }
    router, bias, stacks = _cpu_layer(layers[0], torch)
    if prefill_tokens > 0:  # the full prefill batch, every routed expert dequantised at load
        x = synth.make_tokens(prefill_tokens, seed=7).to(torch.bfloat16)
        ids, _ = _cpu_route(x, router, bias, F, torch)
        used = torch.unique(ids).tolist()
        t_deq = time.perf_counter()
        experts = _cpu_dequant(stacks, used, moe_ref, torch)
        t_deq = time.perf_counter() - t_deq

        def call_p():
            ii, ww = _cpu_route(x, router, bias, F, torch)
            moe_ref.moe_tokens_bf16(x, ii, ww, experts)
        med = timed(call_p)
        flops = synth.prefill_flops(prefill_tokens)
        out["prefill"] = {"tokens": prefill_tokens, "layer_ms_p50": med * 1e3,
                          "TFLOPs": flops / med / 1e12,
                          "dequant_inclusive_layer_ms": (med + t_deq) * 1e3,
                          "sample": f"layer 0 in full, median of {CPU_REPS} reps"}
        log(f"[bench] cpu prefill T={prefill_tokens}: {med * 1e3:.1f} ms/layer "
            f"({flops / med / 1e12:.3f} TFLOP/s) on {threads} threads")
    if block_batches:  # the full block: routed experts plus the gated int4 shared expert
        H = layers[0].experts.hidden_size
        sh = synth.make_experts(1, H, layers[0].experts.intermediate_size, seed=4000)
        shared = tuple(moe_ref.dequant_stack_torch(st.qweight, st.qzeros, st.scales)[0]
                       for st in (sh.gate, sh.up, sh.down))
        sgate = synth.make_shared_gate(H, seed=2500).view(1, H)
        out["block"] = {}
        for T in block_batches:
            x = synth.make_tokens(T, seed=7).to(torch.bfloat16)
            ids, _ = _cpu_route(x, router, bias, F, torch)
            experts = _cpu_dequant(stacks, torch.unique(ids).tolist(), moe_ref, torch)

            def call_b():
                ii, ww = _cpu_route(x, router, bias, F, torch)
                moe_ref.moe_tokens_bf16(x, ii, ww, experts, shared=shared, shared_gate_w=sgate)
            med = timed(call_b)
            out["block"][str(T)] = {"layer_us_p50": med * 1e6,
                                    "sample": f"layer 0 with the shared expert, median of {CPU_REPS} reps"}
    return out


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
