"""Benchmark of the INT4-KV decode path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload ns|c2|c4|c5|c1] [--no-cpu-baseline]
    python bench.py --prefill SQ | --quantize | --model | --stream-probe   (other lines)

A step is one decode token through every layer of the workload: per layer,
quantize-append the new token's K and V into that layer's INT4 cache (in
place, HIP) and run the fused GQA decode attention over the whole context
(HIP). Each layer has its own cache buffers, so a step streams
layers x (cache bytes) from HBM — 576 MiB for the default workload, more than
the 256 MB Infinity Cache holds. The step is captured once in a HIP graph and
replayed; K replays are timed between two events after a device sync.

Default workload "ns": Llama-3.1-8B attention shape (32 query heads, 8 KV
heads, head dim 128, group 32, bf16) at 16K context, 32 layers. Printed: one
JSON line with whole-job algorithmic GB/s (`value`), ms per token, the
attention kernel's roofline (algorithmic bytes / average launch time from HIP
events around every launch, vs 8 TB/s; the counter-measured HBM bytes of the
committed rocprof summary over the same time as traffic_gbs), and the CPU
baseline (the reference's PyTorch CPU path restated in torch, with the C
restatement beside it, each timed on a bounded sample).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "kv-cache-triton_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "INT4-KV decode attn HBM GB/s (% of peak); ms/token, Llama-3.1-8B shape 16K ctx"
HBM_PEAK_GBS = 8000.0

WORKLOADS = {
    # name: (B, Hq, Hkv, D, G, ctx, layers, dtype, ragged)
    "ns": dict(B=1, Hq=32, Hkv=8, D=128, G=32, ctx=16384, layers=32, dtype="bf16", ragged=False,
               desc="llama3.1-8b-decode-16k"),
    "c2": dict(B=1, Hq=32, Hkv=8, D=128, G=32, ctx=4096, layers=32, dtype="bf16", ragged=False,
               desc="llama3.1-8b-decode-4k"),
    "c4": dict(B=8, Hq=64, Hkv=8, D=128, G=32, ctx=32768, layers=80, dtype="bf16", ragged=False,
               desc="llama3.1-70b-shape-b8-decode-32k"),
    "c5": dict(B=16, Hq=25, Hkv=25, D=64, G=32, ctx=1024, layers=48, dtype="f16", ragged=True,
               desc="gpt2-xl-ragged-b16-decode"),
    "c1": dict(B=1, Hq=12, Hkv=12, D=64, G=32, ctx=1024, layers=12, dtype="f32", ragged=False,
               desc="gpt2-small-decode-1k"),
}


def scale_bytes(dtype: str) -> int:
    return 4 if dtype == "f32" else 2


def attn_bytes(w: dict, kv_tokens: int) -> int:
    """Algorithmic HBM bytes of one decode-attention launch: packed K+V codes
    and scales of every attended token, plus q in and o out."""
    ng = -(-w["D"] // w["G"])
    s_sz = 2  # bf16 scales (Llama) or fp16 scales (GPT-2)
    q_sz = 4 if w["dtype"] == "f32" else 2
    return (w["Hkv"] * kv_tokens * (w["D"] + 2 * ng * s_sz)
            + w["B"] * w["Hq"] * w["D"] * 2 * q_sz)


def append_bytes(w: dict) -> int:
    ng = -(-w["D"] // w["G"])
    x_sz = 4 if w["dtype"] == "f32" else 2
    return w["B"] * w["Hkv"] * (2 * w["D"] * x_sz + w["D"] + 2 * ng * 2)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="ns", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=0, help="override the workload's layer count")
    ap.add_argument("--ctx", type=int, default=0, help="override the workload's context length")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of a HIP graph")
    ap.add_argument("--unfused", action="store_true",
                    help="three launches per layer (quantize K, quantize V, attention) instead of the "
                         "fused decode step")
    ap.add_argument("--paged", type=int, default=0, metavar="PAGE_SIZE",
                    help="keep each layer's cache in a block pool of PAGE_SIZE-row pages (>= 64, a power of "
                         "two) addressed through a block table, pages in a seeded random order; 0 = contiguous")
    ap.add_argument("--prefill", type=int, default=0, metavar="SQ",
                    help="time the matrix-core prefill kernel instead: a causal block of SQ query tokens "
                         "over the workload's context (SQ == --ctx: a whole prompt), one JSON line")
    ap.add_argument("--quantize", action="store_true",
                    help="time kvq_quantize / kvq_dequantize on a prompt append of the workload's shape")
    ap.add_argument("--model", action="store_true",
                    help="whole-model decode instead: random-init Llama-3.1-8B (C3), 16K prompt, 64 greedy "
                         "steps over the INT4 cache, each step one HIP graph replay")
    ap.add_argument("--stream-probe", action="store_true",
                    help="the ceiling instead: a streaming-read kernel over the decode step's bytes (one buffer "
                         "per layer, several grids), its per-wave clock stamps, and the decode step's phases "
                         "from the instrumented build of the kernel; one JSON line")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the streaming-read ceiling in the bench line")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="wall budget of the CPU sample (the torch path; the C restatement gets a quarter)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="after the timed region, run a plain device copy of this many MiB (the "
                         "calibration kernel for rocprof FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--traffic-summary", default=os.path.join(ROOT, "profiles", "decode_attn_llama8b_16k_traffic.txt"),
                    help="rocprof counter summary to take roofline.traffic from (if it covers this workload)")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="no GPU work: turn two rocprofv3 --pmc counter_collection.csv files (FETCH_SIZE run, "
                         "WRITE_SIZE run of this script with --calib-copy-mib) into a traffic summary on stdout")
    ap.add_argument("--summarize-trace", metavar="KERNEL_STATS_CSV",
                    help="no GPU work: turn a rocprofv3 --kernel-trace --stats kernel_stats.csv into a summary")
    ap.add_argument("--trace-csv", metavar="KERNEL_TRACE_CSV", default="",
                    help="with --summarize-trace: the run's kernel_trace.csv, for the average over the last "
                         "--trace-tail dispatches of the decode kernel (the bench's timed attention graph)")
    ap.add_argument("--trace-tail", type=int, default=640, help="dispatches averaged by --trace-csv")
    ap.add_argument("--summarize-counters", metavar="COUNTER_CSV",
                    help="no GPU work: per-dispatch, per-wave and per-tile medians of the decode kernel's "
                         "counters in a rocprofv3 --pmc counter_collection.csv")
    ap.add_argument("--tiles-per-wave", type=float, default=1.0,
                    help="64-key tiles each wave of the profiled decode kernel takes (for --summarize-counters)")
    ap.add_argument("--note", default="", help="description line recorded in a counter summary")
    ap.add_argument("--kernel-match", default="decode_attn_",
                    help="kernel-name substring that picks the profiled kernel in --summarize-counters and "
                         "--summarize-pmc (default: the decode kernels; prefill_attn_kernel for --prefill runs)")
    ap.add_argument("--summarize-probe", metavar="PROBE_JSON",
                    help="no GPU work: format the JSON line of a --stream-probe run (ceiling per grid, issue "
                         "cost, decode-step time and phases) as text")
    ap.add_argument("--cmd", default="", help="command line recorded in a summary")
    args = ap.parse_args()

    if args.summarize_pmc:
        print(summarize_pmc(args.summarize_pmc[0], args.summarize_pmc[1], args.calib_copy_mib, args.cmd,
                            args.kernel_match))
        return 0
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.cmd, args.trace_csv, args.trace_tail,
                              args.kernel_match))
        return 0
    if args.summarize_probe:
        print(summarize_probe(args.summarize_probe))
        return 0
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters, args.tiles_per_wave, args.note, args.cmd,
                                 args.kernel_match))
        return 0

    if args.gpus != 1:
        print(f"bench.py: this build runs on exactly one GPU (got --gpus {args.gpus}); the INT4 decode "
              "path is measured on one MI355X (a multi-GPU run would shard KV heads across GPUs with no "
              "exchange inside attention).", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from kvint4 import ops

    w = dict(WORKLOADS[args.workload])
    if args.layers:
        w["layers"] = args.layers
    if args.ctx:
        w["ctx"] = args.ctx
    if args.prefill:
        return prefill_bench(args, w)
    if args.quantize:
        return quantize_bench(args, w)
    if args.model:
        return model_bench(args)
    if args.stream_probe:
        return stream_probe_bench(args, w)
    B, Hq, Hkv, D, G, ctx, L = w["B"], w["Hq"], w["Hkv"], w["D"], w["G"], w["ctx"], w["layers"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    S_cap = ctx + 1
    W_ = ops.packed_width(D, G)
    NG = ops.num_groups(D, G)
    P = args.paged
    if P and (P < 64 or P & (P - 1)):
        print("bench.py: --paged needs a power of two >= 64", file=sys.stderr)
        return 2
    layers, seq_lens, pt = make_layers(w, P, dev, stream)

    pos = seq_lens if seq_lens is not None else ctx
    attended = ctx + 1
    sm_scale = D ** -0.5

    # ragged: each sequence attends its own length plus the new token
    seq_plus = (seq_lens + 1) if seq_lens is not None else None

    # The fused decode step (one launch per layer: the new token's K/V are
    # quantized into the cache and attended along with it) takes group size
    # 32/64/128, and a paged cache 16-bit activations; otherwise, or with
    # --unfused, a layer takes three launches (quantize K, quantize V,
    # attention).
    fused = not args.unfused and G in (32, 64, 128) and not (P and w["dtype"] == "f32")

    def attn(layer):
        if P:
            if fused:
                ops.decode_step_paged(
                    layer["q"], layer["knew"], layer["vnew"], layer["kp"], layer["ks"], layer["vp"], layer["vs"],
                    pt, pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm_scale, out=layer["out"],
                )
            else:
                ops.fused_decode_attention_paged(
                    layer["q"], layer["kp"], layer["ks"], layer["vp"], layer["vs"], pt,
                    n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm_scale,
                    seq_lens=seq_plus, seq_len=None if seq_plus is not None else attended, out=layer["out"],
                )
            return
        if fused:
            ops.decode_step(
                layer["q"], layer["knew"], layer["vnew"], layer["kp"], layer["ks"], layer["vp"], layer["vs"],
                pos, n_kv_heads=Hkv, group_size=G, sm_scale=sm_scale, out=layer["out"],
            )
            return
        ops.fused_decode_attention(
            layer["q"], layer["kp"][:, :, :attended], layer["ks"][:, :, :attended],
            layer["vp"][:, :, :attended], layer["vs"][:, :, :attended],
            n_kv_heads=Hkv, group_size=G, is_causal=False, sm_scale=sm_scale,
            seq_lens=seq_plus, out=layer["out"],
        )

    def step():
        for layer in layers:
            if not fused and P:
                ops.quantize_into_paged(layer["knew"], layer["kp"], layer["ks"], pt, G, pos)
                ops.quantize_into_paged(layer["vnew"], layer["vp"], layer["vs"], pt, G, pos)
            elif not fused:
                ops.quantize_into(layer["knew"], layer["kp"], layer["ks"], G, pos)
                ops.quantize_into(layer["vnew"], layer["vp"], layer["vs"], G, pos)
            attn(layer)

    with torch.cuda.stream(stream):
        for _ in range(max(1, args.warmup)):
            step()
    torch.cuda.synchronize()
    eager_out = [l["out"].clone() for l in layers]

    graph = None
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            step()
        torch.cuda.synchronize()
        # every replay must reproduce the eager result
        for _ in range(3):
            with torch.cuda.stream(stream):
                for l in layers:
                    l["out"].zero_()
                graph.replay()
            torch.cuda.synchronize()
            for l, ref in zip(layers, eager_out):
                if not torch.equal(l["out"], ref):
                    print("bench.py: graph replay differs from the eager step", file=sys.stderr)
                    return 1

    # ---- timed region: K steps ----
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            if graph is not None:
                graph.replay()
            else:
                step()
        e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps

    # ---- attention kernel alone: the L layers' attention launches captured in
    #      one graph, replayed n_rep times between two events on the launch
    #      stream; average duration per launch = elapsed / (n_rep * L) ----
    n_rep = max(2, min(args.steps, 20))
    attn_graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(attn_graph, stream=stream):
        for layer in layers:
            attn(layer)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        attn_graph.replay()  # warm
        a0 = torch.cuda.Event(enable_timing=True)
        a1 = torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        for _ in range(n_rep):
            attn_graph.replay()
        a1.record(stream)
    torch.cuda.synchronize()
    attn_us = a0.elapsed_time(a1) * 1e3 / (n_rep * L)
    for l, ref in zip(layers, eager_out):
        if not torch.equal(l["out"], ref):
            print("bench.py: attention-only graph replay differs from the eager step", file=sys.stderr)
            return 1

    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib, dev, stream)

    kv_tokens = int((seq_lens + 1).sum().item()) if seq_lens is not None else B * attended
    a_bytes = attn_bytes(w, kv_tokens)
    step_bytes = L * (a_bytes + append_bytes(w))
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    # bytes the measured launch moves: the fused step reads the cache's old
    # rows (the new one comes from registers) plus the new K/V rows and writes
    # their codes; the unfused attention launch reads every row
    k_bytes = (attn_bytes(w, kv_tokens - B) + append_bytes(w)) if fused else a_bytes
    achieved = k_bytes / (attn_us * 1e-6) / 1e9

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w["dtype"],
        "data": "synthetic (seeded torch.randn K/V/q, quantized in place by the HIP kernel)",
        "config": {
            "workload": w["desc"], "batch": B, "q_heads": Hq, "kv_heads": Hkv, "head_dim": D,
            "group_size": G, "context": ctx, "layers": L, "ragged": w["ragged"],
            "graph": graph is not None, "fused_step": fused, "paged": P or None,
        },
        "ms_per_token": round(ms_per_step, 5),
        "attn_us_per_layer": round(attn_us, 3),
        "kv_cache_mib": round(L * B * Hkv * attended * 2 * (W_ + NG * 2) / 2**20, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": read_traffic(args.traffic_summary, w),
            "kernel": ("decode_attn_mfma_kernel" if w["dtype"] != "f32" else "decode_attn_valu_kernel")
                      + (" (decode step: append + attention)" if fused else ""),
            "bytes_per_launch": k_bytes,
        },
    }
    traffic = result["roofline"]["traffic"]
    if traffic:
        # HBM bytes the counters saw per launch (FETCH_SIZE + WRITE_SIZE, from the
        # committed summary) over this run's launch time
        result["roofline"]["traffic_gbs"] = round(traffic / (attn_us * 1e-6) / 1e9, 2)

    if not args.no_ceiling and P == 0:
        # the same bytes read by a kernel that does nothing else (one buffer
        # per layer, the best of a few grids): how much of the HBM peak a
        # launch of this size can reach at all
        ceil = stream_ceiling(k_bytes, L, dev, stream, CEILING_GRIDS)
        best = min(ceil, key=lambda r: r["us_per_launch"])
        result["roofline"]["ceiling"] = {
            "achieved": best["gbs"], "unit": "GB/s", "frac_of_peak": round(best["gbs"] / HBM_PEAK_GBS, 4),
            "decode_frac_of_ceiling": round(achieved / best["gbs"], 4), "grid": best["grid"],
            "block": best["block"], "kernarg_preload": best["preload"], "nontemporal": best["nt"],
            "kernel": "stream_read (libkvq_probe.so)",
        }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(w, layers, attended, seq_lens, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


def make_layers(w: dict, P: int, dev, stream):
    """The workload's synthetic per-layer caches, filled by the HIP quantizer
    from seeded torch.randn, plus each layer's new K/V rows, query and output.
    Returns (layers, seq_lens or None, page table or None)."""
    import torch

    from kvint4 import ops

    B, Hq, Hkv, D, G, ctx, L = w["B"], w["Hq"], w["Hkv"], w["D"], w["G"], w["ctx"], w["layers"]
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w["dtype"]]
    sdt = torch.float16 if w["dtype"] != "bf16" else torch.bfloat16  # GPT-2: fp16 scales
    gen = torch.Generator(device=dev).manual_seed(1)
    S_cap = ctx + 1
    W_ = ops.packed_width(D, G)
    NG = ops.num_groups(D, G)
    seq_lens = None
    if w["ragged"]:
        lens = torch.randint(128, ctx + 1, (B,), generator=torch.Generator().manual_seed(4))
        seq_lens = lens.to(dev, torch.int32)
    pt = None
    if P:
        pages = -(-S_cap // P)
        n_blocks = B * pages
        perm = torch.randperm(n_blocks, generator=torch.Generator().manual_seed(5)).to(torch.int32)
        pt = ops.PageTable(perm.view(B, pages).contiguous().to(dev), P, n_blocks)
    layers = []
    with torch.cuda.stream(stream):
        for _ in range(L):
            if P:
                kp = torch.empty(Hkv, pt.num_blocks * P, W_, dtype=torch.uint8, device=dev)
                ks = torch.empty(Hkv, pt.num_blocks * P, NG, dtype=sdt, device=dev)
            else:
                kp = torch.empty(B, Hkv, S_cap, W_, dtype=torch.uint8, device=dev)
                ks = torch.empty(B, Hkv, S_cap, NG, dtype=sdt, device=dev)
            vp = torch.empty_like(kp)
            vs = torch.empty_like(ks)
            for packed, scales in ((kp, ks), (vp, vs)):
                x = torch.randn(B, Hkv, ctx, D, generator=gen, device=dev, dtype=torch.float32).to(tdt)
                if P:
                    ops.quantize_into_paged(x, packed, scales, pt, G, 0)
                else:
                    ops.quantize_into(x, packed, scales, G, 0)
                del x
            layer = dict(
                kp=kp, ks=ks, vp=vp, vs=vs,
                knew=torch.randn(B, Hkv, 1, D, generator=gen, device=dev, dtype=torch.float32).to(tdt),
                vnew=torch.randn(B, Hkv, 1, D, generator=gen, device=dev, dtype=torch.float32).to(tdt),
                q=torch.randn(B, Hq, 1, D, generator=gen, device=dev, dtype=torch.float32).to(tdt),
                out=torch.empty(B, Hq, 1, D, device=dev, dtype=tdt),
            )
            layers.append(layer)
    torch.cuda.synchronize()
    return layers, seq_lens, pt


# (grid, block) of the streaming-read probe: whole-GPU fills from one
# workgroup per CU to eight
PROBE_GRIDS = ((256, 256), (256, 512), (256, 1024), (512, 256), (512, 512), (1024, 256), (1024, 512),
               (2048, 256), (2048, 512))
CEILING_GRIDS = ((256, 512), (512, 256), (1024, 256), (2048, 256), (2048, 512))


def probe_lib():
    """libkvq_probe.so: the streaming-read probe and the phase-stamped build of
    the decode kernels (measurement only; never used by the product path)."""
    import ctypes

    from kvint4 import _native as nat

    path = os.path.join(ROOT, "kv-cache-triton_amd", "kvint4", "libkvq_probe.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(path)
    prod = nat.lib()
    for name in ("kvq_decode_step", "kvq_decode_attn_num_splits", "kvq_decode_attn_workspace_bytes", "kvq_last_error"):
        fn = getattr(lib, name)
        fn.restype = getattr(prod, name).restype
        fn.argtypes = getattr(prod, name).argtypes
    for name in ("kvq_probe_stream_read", "kvq_probe_stream_read_preload", "kvq_probe_stream_read_preload_nt"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                       ctypes.c_void_p]
    lib.kvq_probe_stream_read_padded.restype = ctypes.c_int
    lib.kvq_probe_stream_read_padded.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                                                 ctypes.c_void_p, ctypes.c_void_p]
    lib.kvq_probe_set_phase_stamps.restype = ctypes.c_int
    lib.kvq_probe_set_phase_stamps.argtypes = [ctypes.c_void_p]
    return lib


def stream_ceiling(nbytes: int, L: int, dev, stream, grids, keep=None) -> list:
    """Streaming read of nbytes (rounded up to 16) from each of L buffers, one
    launch per buffer captured in a HIP graph and replayed 20 times between
    two events on the launch stream: per (grid, block) and per build of the
    read (preload False: the wave loads its arguments from memory; True: the
    hardware preloads them into SGPRs; nt: preloaded, and the loads carry the
    nontemporal hint), the average launch time and GB/s over nbytes."""
    import torch

    lib = probe_lib()
    n = -(-nbytes // 16) * 16
    g = torch.Generator(device=dev).manual_seed(7)
    bufs = [torch.randint(0, 255, (n,), dtype=torch.uint8, device=dev, generator=g) for _ in range(L)]
    sink = torch.zeros(1 << 20, dtype=torch.int32, device=dev)  # >= any grid below (one word per workgroup)
    out = []
    for (grid, block), (preload, nt) in ((gb, v) for gb in grids for v in ((False, False), (True, False), (True, True))):
        # larger buffers: more workgroups, so that each thread keeps at most
        # 20 pieces in flight (no register spills)
        while -(-(n // 16) // (grid * block)) > 20:
            grid *= 2
        read = (lib.kvq_probe_stream_read_preload_nt if nt else
                lib.kvq_probe_stream_read_preload if preload else lib.kvq_probe_stream_read)
        graph = torch.cuda.CUDAGraph()
        per = 0
        with torch.cuda.graph(graph, stream=stream):
            for b in bufs:
                per = read(b.data_ptr(), n, grid, block, sink.data_ptr(), None, stream.cuda_stream)
        if per <= 0:
            continue
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            for _ in range(3):
                graph.replay()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(20):
                graph.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (20 * L)
        out.append({"grid": grid, "block": block, "preload": preload, "nt": nt, "pieces_per_thread": per,
                    "us_per_launch": round(us, 3), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)})
    if keep is not None:
        keep.extend(bufs)
    return out


def _dist(vals) -> dict:
    import numpy as np

    v = np.sort(np.asarray(vals, dtype=np.float64))
    if v.size == 0:
        return {}
    q = lambda f: round(float(v[min(v.size - 1, int(f * v.size))]), 0)
    return {"n": int(v.size), "min": q(0.0), "p10": q(0.1), "med": q(0.5), "p90": q(0.9), "max": round(float(v[-1]), 0)}


def stream_probe_bench(args, w: dict) -> int:
    """--stream-probe: what a launch of the decode step's size can reach, and
    where the decode step's time goes. Prints one JSON line:
    - stream: the streaming-read kernel over the step's bytes, per grid;
    - stream_phases_ns: its per-wave clock stamps on a cold buffer (entry, all
      loads issued, first and last data arrived), ns after the first wave;
    - decode_step: the product kernel's launch time (graph of the workload's
      layers, as the bench line) and its fraction of the best read;
    - decode_phases_ns: the instrumented build of the same kernel on a cold
      layer, per point (entry, loads issued, keys / values of the first tile
      arrived, tile loop done, workgroup fold done, partial acknowledged,
      arrival counted, merge start, merge inputs arrived, merged, exit)."""
    import numpy as np
    import torch

    from kvint4 import _native as nat
    from kvint4 import ops

    if w["dtype"] == "f32" or w["ragged"]:
        print("bench.py: --stream-probe takes a 16-bit workload with one length for the batch", file=sys.stderr)
        return 2
    B, Hq, Hkv, D, G, ctx, L = w["B"], w["Hq"], w["Hkv"], w["D"], w["G"], w["ctx"], w["layers"]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    lib = probe_lib()
    nbytes = attn_bytes(w, B * ctx) + append_bytes(w)  # what one decode-step launch must move
    keep = []
    stream_rows = stream_ceiling(nbytes, L, dev, stream, PROBE_GRIDS, keep)
    best = min(stream_rows, key=lambda r: r["us_per_launch"])

    # per-wave stamps of the read on a cold buffer (the other buffers read first);
    # the build without argument preload, which starts its waves the way the
    # decode kernel does
    n = -(-nbytes // 16) * 16
    grid, block = 256, 512
    waves = grid * (block // 64)
    st = torch.zeros(grid * 16 * 4, dtype=torch.int64, device=dev)
    sink = torch.zeros(grid, dtype=torch.int32, device=dev)
    with torch.cuda.stream(stream):
        for b in keep[1:]:
            lib.kvq_probe_stream_read(b.data_ptr(), n, grid, block, sink.data_ptr(), None, stream.cuda_stream)
        rc = lib.kvq_probe_stream_read(keep[0].data_ptr(), n, grid, block, sink.data_ptr(), st.data_ptr(),
                                       stream.cuda_stream)
    torch.cuda.synchronize()
    if rc <= 0:
        print("bench.py: stamped streaming read did not launch", file=sys.stderr)
        return 1
    s = st.view(grid, 16, 4)[:, : block // 64].reshape(waves, 4).cpu().numpy()
    t0 = s[:, 0].min()
    names = ("entry", "loads_issued", "first_arrived", "all_arrived")
    stream_phases = {nm: _dist((s[:, k] - t0) * 10.0) for k, nm in enumerate(names)}

    # issue cost: the same read (grid 256 x 512, 10 pieces per thread) with N
    # dependent VALU instructions before (or after) its loads
    issue = []
    if n <= 256 * 512 * 10 * 16:
        for pad, after in ((0, 0), (256, 0), (512, 0), (1024, 0), (2048, 0), (512, 1), (2048, 1)):
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                for b in keep:
                    rc = lib.kvq_probe_stream_read_padded(b.data_ptr(), n, pad, after, sink.data_ptr(),
                                                          stream.cuda_stream)
            if rc != 0:
                continue
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                for _ in range(3):
                    graph.replay()
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(20):
                    graph.replay()
                e1.record(stream)
            torch.cuda.synchronize()
            issue.append({"valu_instructions": pad, "placed": "after loads" if after else "before loads",
                          "us_per_launch": round(e0.elapsed_time(e1) * 1e3 / (20 * len(keep)), 3)})
    del keep

    # the decode step: product kernel timing, then the instrumented build's phases
    layers, _, _ = make_layers(w, 0, dev, stream)
    sm_scale = D ** -0.5

    def step():
        for layer in layers:
            ops.decode_step(layer["q"], layer["knew"], layer["vnew"], layer["kp"], layer["ks"], layer["vp"],
                            layer["vs"], ctx, n_kv_heads=Hkv, group_size=G, sm_scale=sm_scale, out=layer["out"])

    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        graph.replay()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(20):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    dec_us = e0.elapsed_time(e1) * 1e3 / (20 * L)
    dec_bytes = attn_bytes(w, B * ctx) + append_bytes(w)

    qd, sd = nat.DTYPE_CODE[layers[0]["q"].dtype], nat.DTYPE_CODE[layers[0]["ks"].dtype]
    cap = int(layers[0]["kp"].shape[2])
    ns = lib.kvq_decode_attn_num_splits(B, Hq, Hkv, 1, D, ctx + 1, qd, sd, ops._num_cus(dev))
    ws_bytes = lib.kvq_decode_attn_workspace_bytes(B, Hq, Hkv, 1, D, qd, sd, ns)
    ws = torch.zeros(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    n_wg = 8 * ns * -(-(B * Hkv * -(-(Hq // Hkv) // 8)) // 8)  # launched workgroups (one row chunk per unit)
    ph = torch.zeros(n_wg * 16 * 16, dtype=torch.int64, device=dev)

    def stamped(layer) -> None:
        rc = lib.kvq_decode_step(
            layer["q"].data_ptr(), qd, nat.i64_array(layer["q"].stride()),
            layer["knew"].data_ptr(), nat.i64_array(layer["knew"].stride()),
            layer["vnew"].data_ptr(), nat.i64_array(layer["vnew"].stride()),
            layer["kp"].data_ptr(), nat.i64_array(layer["kp"].stride()[:3]),
            layer["ks"].data_ptr(), nat.i64_array(layer["ks"].stride()[:3]),
            layer["vp"].data_ptr(), nat.i64_array(layer["vp"].stride()[:3]),
            layer["vs"].data_ptr(), nat.i64_array(layer["vs"].stride()[:3]),
            sd, layer["out"].data_ptr(), nat.i64_array(layer["out"].stride()),
            B, Hq, Hkv, D, G, cap, None, ctx, float(sm_scale), ns, ws.data_ptr(), ws.numel(),
            stream.cuda_stream)
        if rc != 0:
            raise RuntimeError(f"instrumented kvq_decode_step: {lib.kvq_last_error().decode()}")

    with torch.cuda.stream(stream):
        for layer in layers[1:]:
            stamped(layer)  # stamps off (null buffer): evicts layer 0's cache from the caches
    torch.cuda.synchronize()
    if lib.kvq_probe_set_phase_stamps(ph.data_ptr()) != 0:
        raise RuntimeError("kvq_probe_set_phase_stamps failed")
    with torch.cuda.stream(stream):
        stamped(layers[0])
    torch.cuda.synchronize()
    lib.kvq_probe_set_phase_stamps(None)
    a = ph.view(n_wg, 16, 16).cpu().numpy()
    nz = a[:, :, 0] > 0
    t0 = a[:, :, 0][nz].min()
    points = ("entry", "loads_issued", "keys_arrived", "values_arrived", "tile_loop_done", "wg_fold_done",
              "partial_acked", "arrival_counted", "merge_start", "merge_inputs_arrived", "merged", "exit")
    dec_phases = {}
    for k, nm in enumerate(points):
        v = a[:, :, k]
        v = v[v > 0]
        if v.size:
            dec_phases[nm] = _dist((v - t0) * 10.0)
    result = {
        "metric": "streaming-read ceiling and decode-step phases (one MI355X)",
        "workload": w["desc"], "bytes_per_launch": nbytes, "layers": L,
        "stream": stream_rows, "best": best,
        "stream_phases_ns": dict(stream_phases, grid=grid, block=block),
        "issue_cost": issue,
        "decode_step": {"us_per_launch": round(dec_us, 3), "gbs": round(dec_bytes / (dec_us * 1e-6) / 1e9, 1),
                        "frac_of_peak": round(dec_bytes / (dec_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                        "frac_of_best_read": round(best["us_per_launch"] / dec_us, 4), "n_split": int(ns)},
        "decode_phases_ns": dec_phases,
    }
    print(json.dumps(result), flush=True)
    return 0


MFMA_BF16_PEAK_TFS = 2500.0  # MI355X dense bf16 / fp16 matrix peak


def calibration_copy(mib: int, dev, stream) -> None:
    """An elementwise kernel that reads and writes mib MiB, three times (bitwise
    not of uint8; a same-dtype copy_ would go to a DMA engine, which kernel
    counters do not see): the reference point that scales rocprof's FETCH_SIZE
    / WRITE_SIZE readings to bytes."""
    import torch

    n = mib << 20
    src_buf = torch.zeros(n, dtype=torch.uint8, device=dev)
    dst_buf = torch.empty_like(src_buf)
    with torch.cuda.stream(stream):
        for _ in range(3):
            torch.bitwise_not(src_buf, out=dst_buf)
    torch.cuda.synchronize()
    del src_buf, dst_buf


def prefill_bench(args, w: dict) -> int:
    """Attention of a causal block of Sq query tokens over the workload's
    context (Sk keys, the block's own tokens last) on kvq_prefill_attn, with
    the dequantize + flash SDPA route timed beside it. Algorithmic work: QK
    and PV over the admissible (bottom-right causal) key range, 4 * D flops
    per (query head, query, key) pair. Four layers' caches are cycled."""
    import torch

    from kvint4 import ops

    B, Hq, Hkv, D, G, Sk = w["B"], w["Hq"], w["Hkv"], w["D"], w["G"], w["ctx"]
    Sq = min(args.prefill, Sk)
    if w["dtype"] == "f32" or w["ragged"]:
        print("bench.py: --prefill takes a 16-bit workload with one length for the batch", file=sys.stderr)
        return 2
    dt = torch.bfloat16 if w["dtype"] == "bf16" else torch.float16
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0)
    layers = []
    for _ in range(4):
        kp, ks = ops.quantize(torch.randn(B, Hkv, Sk, D, device=dev, generator=gen).to(dt), G, dt)
        vp, vs = ops.quantize(torch.randn(B, Hkv, Sk, D, device=dev, generator=gen).to(dt), G, dt)
        q = torch.randn(B, Hq, Sq, D, device=dev, generator=gen).to(dt)
        layers.append((q, kp, ks, vp, vs, torch.empty_like(q)))
    kw = dict(n_kv_heads=Hkv, group_size=G, is_causal=True, sm_scale=D ** -0.5)

    def step():
        for q, kp, ks, vp, vs, o in layers:
            ops.prefill_attention(q, kp, ks, vp, vs, out=o, **kw)

    def dense_step():
        for q, kp, ks, vp, vs, o in layers:
            ops.dense_attention_over_quantized(q, kp, ks, vp, vs, **kw)

    def timed(fn, n):
        for _ in range(max(1, args.warmup)):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / (n * len(layers))  # ms per layer

    steps = max(1, min(args.steps, 20))
    ms = timed(step, steps)
    ms_dense = timed(dense_step, max(1, steps // 2))
    err = (layers[0][5].float() - ops.dense_attention_over_quantized(*layers[0][:5], **kw).float()).abs().max().item()
    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib, dev, torch.cuda.current_stream(dev))
    pairs = sum(min(Sk, Sk - Sq + i + 1) for i in range(Sq))  # admissible (query, key) pairs per head
    flops = 4.0 * B * Hq * D * pairs
    tfs = flops / (ms * 1e-3) / 1e12
    print(json.dumps({
        "metric": "INT4-KV prefill attention TFLOP/s (matrix cores)", "value": round(tfs, 1), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": w["dtype"],
        "data": "synthetic (seeded torch.randn K/V/q, quantized by the HIP kernel)",
        "config": {"workload": f"{w['desc'].replace('decode', 'prefill')}", "batch": B, "q_heads": Hq,
                   "kv_heads": Hkv, "head_dim": D, "group_size": G, "context": Sk, "query_tokens": Sq,
                   "causal": True},
        "roofline": {"bound": "mfma", "achieved": round(tfs, 1), "peak": MFMA_BF16_PEAK_TFS, "unit": "TFLOP/s",
                     "frac": round(tfs / MFMA_BF16_PEAK_TFS, 4), "traffic": None, "kernel": "prefill_attn_kernel"},
        "dequant_flash_ms_per_layer": round(ms_dense, 4), "max_abs_vs_dequant_flash": err,
    }), flush=True)
    return 0


def quantize_bench(args, w: dict) -> int:
    """The quantizer on a prompt append: x [B, Hkv, ctx, D] of the workload's
    activation dtype quantized into fresh cache tensors (`kvq_quantize`, the
    path's a1 row), and the same codes dequantized back (`kvq_dequantize`).
    Bytes per launch: the input read plus codes and scales written (quantize),
    codes and scales read plus the output written (dequantize). Enough
    buffers rotate that one round exceeds the 256 MB Infinity Cache; the
    launches are captured in a HIP graph, replayed untimed at least 40 times,
    then timed with events on the launch stream (mean per launch over the
    timed replays, and their range)."""
    import math

    import torch

    from kvint4 import ops

    B, Hkv, D, G, S = w["B"], w["Hkv"], w["D"], w["G"], w["ctx"]
    if w["dtype"] == "f32":
        print("bench.py: --quantize takes a 16-bit workload", file=sys.stderr)
        return 2
    dt = torch.bfloat16 if w["dtype"] == "bf16" else torch.float16
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream(dev)
    W_, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    n = B * Hkv * S
    x_bytes, code_bytes = n * D * 2, n * (W_ + 2 * NG)
    nbuf = max(2, math.ceil((512 << 20) / (x_bytes + code_bytes)))
    gen = torch.Generator(device=dev).manual_seed(5)
    xs = [(torch.randn(B, Hkv, S, D, device=dev, generator=gen) * 3).to(dt) for _ in range(nbuf)]
    pk = [torch.empty(B, Hkv, S, W_, device=dev, dtype=torch.uint8) for _ in range(nbuf)]
    sc = [torch.empty(B, Hkv, S, NG, device=dev, dtype=dt) for _ in range(nbuf)]
    outs = [torch.empty(B, Hkv, S, D, device=dev, dtype=dt) for _ in range(nbuf)]

    def quant_round():
        for j in range(nbuf):
            ops.quantize_into(xs[j], pk[j], sc[j], G)

    lib = ops.nat.lib()

    def dequant_round():
        # the kernel launch of ops.dequantize, into preallocated outputs
        for j in range(nbuf):
            rc = lib.kvq_dequantize(
                pk[j].data_ptr(), ops.nat.i64_array(pk[j].stride()[:3]),
                sc[j].data_ptr(), ops.nat.DTYPE_CODE[dt], ops.nat.i64_array(sc[j].stride()[:3]),
                B, Hkv, S, G, NG, outs[j].data_ptr(), ops.nat.DTYPE_CODE[dt], ops.nat.i64_array(outs[j].stride()),
                D, stream.cuda_stream)
            ops.nat.check(rc, "kvq_dequantize")

    rounds = 4

    def timed(fn) -> float:
        with torch.cuda.stream(stream):
            for _ in range(max(1, args.warmup)):
                fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(rounds):
                fn()
        torch.cuda.synchronize()
        # At least 40 untimed replays (tens of ms of launches): for the first
        # tens of ms of sustained launches after an idle period these kernels
        # run up to 40 % slower, on this part, than in the steady state after.
        with torch.cuda.stream(stream):
            for _ in range(max(40, args.warmup)):
                g.replay()
        torch.cuda.synchronize()
        reps = max(1, min(args.steps, 20))
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        with torch.cuda.stream(stream):  # a graph replays on the current stream
            ev[0].record(stream)
            for i in range(reps):
                g.replay()
                ev[i + 1].record(stream)
        torch.cuda.synchronize()
        per = [ev[i].elapsed_time(ev[i + 1]) * 1e3 / (rounds * nbuf) for i in range(reps)]
        # µs per launch: the mean over every timed replay, and the range of the replays' means
        return sum(per) / reps, min(per), max(per)

    us_q, q_lo, q_hi = timed(quant_round)
    us_dq, dq_lo, dq_hi = timed(dequant_round)
    # round-trip sanity of the timed outputs: |dequant(quant(x)) - x| is half a
    # scale step, plus the roundings of the stored scale and of the output
    # (0.6 of a step bounds both)
    x0 = xs[0].float().view(n, NG, G)
    err = (outs[0].float().view(n, NG, G) - x0).abs().amax(-1)
    rt_ok = bool((err <= sc[0].float().abs().view(n, NG) * 0.6).all().item())
    if args.calib_copy_mib:
        calibration_copy(args.calib_copy_mib, dev, stream)
    gbs_q = (x_bytes + code_bytes) / (us_q * 1e-6) / 1e9
    gbs_dq = (x_bytes + code_bytes) / (us_dq * 1e-6) / 1e9
    print(json.dumps({
        "metric": "INT4 quantize of a prompt's K (or V) rows, HBM GB/s", "value": round(gbs_q, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": max(1, min(args.steps, 20)), "warmup": args.warmup, "us_per_launch": round(us_q, 3),
        "us_per_launch_range": [round(q_lo, 3), round(q_hi, 3)],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": w["dtype"],
        "data": "synthetic (seeded torch.randn * 3)",
        "config": {"workload": f"{w['desc'].replace('decode', 'prompt-append')}", "shape": [B, Hkv, S, D],
                   "group_size": G, "rotating_buffers": nbuf},
        "roofline": {"bound": "hbm", "achieved": round(gbs_q, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs_q / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "quantize_vec_kernel",
                     "bytes_per_launch": x_bytes + code_bytes},
        "dequantize": {"gbs": round(gbs_dq, 1), "us_per_launch": round(us_dq, 3),
                       "us_per_launch_range": [round(dq_lo, 3), round(dq_hi, 3)],
                       "frac": round(gbs_dq / HBM_PEAK_GBS, 4), "kernel": "dequantize_vec_kernel"},
        "round_trip_within_half_scale": rt_ok,
    }), flush=True)
    return 0 if rt_ok else 1


def model_bench(args) -> int:
    """Whole-model decode at the C3 configuration: random-init Llama-3.1-8B in
    bf16 (weights ~N(0, 0.02) from the HF initialiser, seed 2), a 16384-token
    uniform random prompt (seed 2), prefill through the swapped attention
    modules (INT4 cache, matrix-core prefill kernel), then 64 greedy steps:
    2 eager warmup steps, then one HIP graph replay per token
    (kvint4.llama3.graph_decode). ms/token is the replays' event time over
    their count. Eager HF decoding of the same cache is timed beside it. The
    roofline is that of the whole step: every weight but the embedding table is
    read once per token (bf16 GEMV), plus each layer's INT4 K/V."""
    import torch
    from transformers import LlamaConfig, LlamaForCausalLM

    from kvint4.llama3.graph_decode import GraphedGreedyDecoder
    from kvint4.llama3.kv_cache import QuantizedKVCache
    from kvint4.llama3.llama3_quant import replace_llama_attention_with_quantized

    prompt_len, total, warm, eager_steps = 16384, 64, 2, 8
    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                      num_attention_heads=32, num_key_value_heads=8, rope_theta=500000.0,
                      max_position_embeddings=131072, rms_norm_eps=1e-5, initializer_range=0.02,
                      tie_word_embeddings=False)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    torch.manual_seed(2)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(dev):
            model = LlamaForCausalLM(cfg).eval()
    finally:
        torch.set_default_dtype(prev)
    model.set_attn_implementation("sdpa")
    replace_llama_attention_with_quantized(model, group_size=32)
    print("bench.py --model: model initialised", file=sys.stderr, flush=True)
    prompt = torch.randint(0, cfg.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(2)).to(dev)
    cache = QuantizedKVCache(group_size=32, reserve_tokens=prompt_len + total + eager_steps + 64)
    with torch.no_grad():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        out = model(input_ids=prompt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        torch.cuda.synchronize()
        prefill_s = time.perf_counter() - t0
        nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        del out
        # eager HF decoding of the same cache (Python overhead included)
        eager = []
        for _ in range(eager_steps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True, logits_to_keep=1)
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
            torch.cuda.synchronize()
            eager.append(time.perf_counter() - t0)
    print(f"bench.py --model: prefill {prefill_s:.2f} s, eager decode done", file=sys.stderr, flush=True)
    dec = GraphedGreedyDecoder(model, cache, nxt, max_new_tokens=total, warmup_steps=warm)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    toks = dec.run()
    e1.record()
    torch.cuda.synchronize()
    replays = total - warm
    ms_tok = e0.elapsed_time(e1) / replays
    kv_tokens = cache.get_seq_length(0)
    assert kv_tokens == prompt_len + eager_steps + total, kv_tokens
    weight_bytes = sum(p.numel() * p.element_size() for n, p in model.named_parameters() if "embed_tokens" not in n)
    w = WORKLOADS["ns"]
    mid = prompt_len + eager_steps + (warm + total) // 2  # keys attended by the middle replay
    kv_bytes = cfg.num_hidden_layers * (attn_bytes(w, mid) + append_bytes(w))
    gbs = (weight_bytes + kv_bytes) / (ms_tok * 1e-3) / 1e9
    eager_ms = 1e3 * sorted(eager)[len(eager) // 2]
    print(json.dumps({
        "metric": "Llama-3.1-8B decode ms/token, INT4 KV cache, 16K prompt", "value": round(ms_tok, 4),
        "unit": "ms/token", "n_gpus": 1, "steps": replays, "warmup": warm, "ms_per_step": round(ms_tok, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (random-init weights ~N(0,0.02), seed 2; uniform random 16384-token prompt, seed 2)",
        "config": {"workload": "llama3.1-8b-c3-prefill16k-greedy64", "batch": 1, "layers": 32, "hidden": 4096,
                   "q_heads": 32, "kv_heads": 8, "ffn": 14336, "vocab": 128256, "group_size": 32,
                   "prompt": prompt_len, "graph": True},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole decode step (bf16 weights once + INT4 K/V of every layer)",
                     "bytes_per_step": int(weight_bytes + kv_bytes)},
        "eager_hf_ms_per_token": round(eager_ms, 3), "prefill_s": round(prefill_s, 3),
        "kv_cache_mib": round(cache.nbytes() / 2**20, 2),
        "tokens_head": toks[0, :8].tolist(),
    }), flush=True)
    return 0


def _counter_medians(path: str) -> dict:
    """Median per (kernel name, counter) of a rocprofv3 counter_collection.csv."""
    import csv
    import statistics

    vals: dict = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            key = (row["Kernel_Name"], row["Counter_Name"])
            vals.setdefault(key, []).append(float(row["Counter_Value"]))
    return {k: (statistics.median(v), len(v)) for k, v in vals.items()}


def _pick(med: dict, counter: str, want) -> tuple:
    """(kernel name, median, dispatches) of the kernel matching `want` with the
    largest median reading of `counter`."""
    best = None
    for (name, cname), (m, n) in med.items():
        if cname == counter and want(name) and (best is None or m > best[1]):
            best = (name, m, n)
    if best is None:
        raise SystemExit(f"no kernel with counter {counter} matched in the summary input")
    return best


def summarize_pmc(fetch_csv: str, write_csv: str, calib_mib: int, cmd: str, match: str = "decode_attn_") -> str:
    """Traffic summary: the attention kernel's (name containing `match`)
    FETCH_SIZE and WRITE_SIZE (KiB per dispatch, median over dispatches), each
    scaled by expected / measured of the same counter on the calibration kernel
    (bitwise not over calib_mib MiB, which reads and writes calib_mib MiB)."""
    if calib_mib <= 0:
        raise SystemExit("--summarize-pmc needs --calib-copy-mib (the size the profiled run copied)")
    is_attn = lambda n: match in n and "merge" not in n
    is_copy = lambda n: "bitwise_not" in n
    out = []
    res = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        med = _counter_medians(path)
        an, av, ad = _pick(med, counter, is_attn)
        cn, cv, cd = _pick(med, counter, is_copy)
        expect_kib = calib_mib * 1024.0
        factor = expect_kib / cv if cv > 0 else float("nan")
        res[counter] = av * factor
        out.append(f"{counter}: {'attention' if 'attn' in match else 'kernel'} {av:.1f} KiB/dispatch "
                   f"(median of {ad}; {an[:80]})")
        out.append(f"{counter}: calibration copy {cv:.1f} KiB/dispatch for {expect_kib:.0f} KiB moved "
                   f"(median of {cd}; {cn[:80]}) -> factor {factor:.4f}")
    total = (res["FETCH_SIZE"] + res["WRITE_SIZE"]) * 1024.0
    out.append(f"traffic_bytes_per_launch: {total:.0f}")
    out.append(f"fetch_bytes_per_launch: {res['FETCH_SIZE'] * 1024.0:.0f}")
    out.append(f"write_bytes_per_launch: {res['WRITE_SIZE'] * 1024.0:.0f}")
    return "\n".join([f"command: {cmd}" if cmd else "command: (not recorded)"] + out)


def summarize_counters(path: str, tiles_per_wave: float, note: str, cmd: str, match: str = "decode_attn_") -> str:
    """Counter summary of the profiled kernel (of the kernels whose name
    contains `match`, the one with the most dispatches): for each counter its
    median per dispatch, that divided by the dispatch's waves (Grid_Size / 64),
    and by tiles_per_wave; plus VALU issue = SQ_ACTIVE_INST_VALU /
    SQ_WAVE_CYCLES when both were collected."""
    import csv
    import statistics

    vals: dict = {}
    grids: dict = {}
    with open(path) as f:
        for row in csv.DictReader(f):
            name = row["Kernel_Name"]
            if match not in name:
                continue
            vals.setdefault(name, {}).setdefault(row["Counter_Name"], []).append(float(row["Counter_Value"]))
            grids.setdefault(name, []).append(int(row["Grid_Size"]))
    if not vals:
        raise SystemExit(f"no kernel matching {match!r} in the counter input")
    name = max(vals, key=lambda n: len(grids[n]))
    waves = statistics.median(grids[name]) / 64.0
    out = [f"command: {cmd}" if cmd else "command: (not recorded)", f"kernel: {name[:110]}"]
    if note:
        out.append(note)
    out.append(f"{'counter':<22} {'median/dispatch':>16} {'per wave':>10} {'per tile':>10}  (dispatches)")
    med = {}
    for c in sorted(vals[name]):
        m = statistics.median(vals[name][c])
        med[c] = m
        out.append(f"{c:<22} {m:16.0f} {m / waves:10.1f} {m / waves / tiles_per_wave:10.1f}  "
                   f"({len(vals[name][c])})")
    if "SQ_ACTIVE_INST_VALU" in med and med.get("SQ_WAVE_CYCLES"):
        out.append(f"VALU issue fraction SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES = "
                   f"{med['SQ_ACTIVE_INST_VALU'] / med['SQ_WAVE_CYCLES']:.3f}")
    return "\n".join(out)


def summarize_probe(path: str) -> str:
    """Text form of a --stream-probe JSON line (its last line in `path`)."""
    d = json.loads(open(path).read().strip().splitlines()[-1])
    best = d["best"]
    out = [f"streaming read of {d['bytes_per_launch']} B per launch, {d['layers']} buffers, graph of "
           f"{d['layers']} launches x 20 replays:"]
    for r in d["stream"]:
        pl = ("preloaded, nt" if r.get("nt") else "preloaded args") if r.get("preload") else "args from memory"
        out.append(f"  grid {r['grid']:5d} x {r['block']:4d}  {r['pieces_per_thread']:2d} x 16 B per thread  "
                   f"{pl:<16}  {r['us_per_launch']:7.3f} us/launch  {r['gbs']:7.1f} GB/s")
    for r in d.get("issue_cost", []):
        out.append(f"  grid   256 x  512  10 x 16 B per thread  args from memory  {r['valu_instructions']:4d} VALU "
                   f"{r['placed']:<12}  {r['us_per_launch']:7.3f} us/launch")
    dec = d["decode_step"]
    out.append(f"decode step (product kernel, same graph timing): {dec['us_per_launch']:.3f} us/launch = "
               f"{dec['gbs']:.1f} GB/s, {dec['frac_of_best_read']:.3f} of the best read "
               f"({best['us_per_launch']:.3f} us)")

    def table(title, phases, keys):
        rows = [f"{title:<60}{'min':>6}{'med':>8}{'p90':>8}{'max':>8}"]
        for k in keys:
            if k in phases:
                v = phases[k]
                label = f"  {k:<22} (n {v['n']:4d})" if "n" in v else f"  {k:<22}"
                rows.append(f"{label:<60}{v['min']:6.0f}{v['med']:8.0f}{v['p90']:8.0f}{v['max']:8.0f}")
        return rows

    sp = d["stream_phases_ns"]
    out += table(f"streaming read, per-wave stamps (grid {sp['grid']} x {sp['block']}, args from memory), ns:", sp,
                 ("entry", "loads_issued", "first_arrived", "all_arrived"))
    out += table("decode step, instrumented build (libkvq_probe.so), per wave, ns:", d["decode_phases_ns"],
                 list(d["decode_phases_ns"]))
    return "\n".join(out)


def summarize_trace(stats_csv: str, cmd: str, trace_csv: str = "", tail: int = 640,
                    match: str = "decode_attn_") -> str:
    """Per-kernel call count and average / min / max duration from a rocprofv3
    --stats kernel_stats.csv, kvq kernels first. With the run's
    kernel_trace.csv, also the average over the last `tail` dispatches of the
    kernel (name containing `match`) with the most dispatches: in a bench.py
    run those are its timed attention-graph replays (steps x layers launches),
    the launches its roofline figure averages; the whole-run average also
    holds eager warm-up launches and the step graph's replays."""
    import csv

    rows = list(csv.DictReader(open(stats_csv)))
    rows.sort(key=lambda r: ("kvq::" not in r["Name"], -float(r["TotalDurationNs"])))
    out = [f"command: {cmd}" if cmd else "command: (not recorded)",
           f"{'calls':>7} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}  kernel"]
    for r in rows[:12]:
        out.append(f"{int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.3f} {float(r['MinNs']) / 1e3:9.3f} "
                   f"{float(r['MaxNs']) / 1e3:9.3f} {float(r['Percentage']):6.2f}  {r['Name'][:110]}")
    if trace_csv:
        disp: dict = {}
        for r in csv.DictReader(open(trace_csv)):
            if match in r["Kernel_Name"]:
                disp.setdefault(r["Kernel_Name"], []).append(
                    (int(r["Start_Timestamp"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])))
        if disp:
            name, ds = max(disp.items(), key=lambda kv: len(kv[1]))
            ds.sort()
            last = [d for _, d in ds[-tail:]]
            out.append(f"last {len(last)} of {len(ds)} dispatches of {name[:80]}: average "
                       f"{sum(last) / len(last) / 1e3:.3f} us (min {min(last) / 1e3:.3f}, max {max(last) / 1e3:.3f})")
    return "\n".join(out)


def read_traffic(path: str, w: dict):
    """traffic_bytes_per_launch from a committed summary, if it was made for
    this workload (its command names the same --workload and no other context)."""
    try:
        text = open(path).read()
    except OSError:
        return None
    cmd = next((l for l in text.splitlines() if l.startswith("command:")), "")
    wl = "ns" if "--workload" not in cmd else cmd.split("--workload", 1)[1].split()[0]
    if WORKLOADS.get(wl, {}).get("desc") != w["desc"] or "--ctx" in cmd:
        return None
    for line in text.splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(w: dict, layers: list, attended: int, seq_lens, budget_s: float) -> dict:
    """Time the reference's PyTorch CPU path on the host cores: per layer-step,
    quantize the new K/V row, torch.cat the four tensors onto that layer's cache
    (models/llama3/kv_cache.py:96-101), dequantize the whole cache and attend
    with repeat_interleave + SDPA (oracle/kvq_torch.py restates each step). The
    sample rotates over every layer of the workload (each with its own cache,
    copied from the GPU), as the GPU step does, for about `budget_s` seconds,
    with torch's intra-op thread count (OMP_NUM_THREADS, the process's CPU
    share). The C restatement (oracle/kvq_ref.c, OpenMP, no concatenation) is
    timed beside it on a shorter sample and reported as `c_port`."""
    import numpy as np
    import torch

    from oracle import kvq_ref as R
    from oracle import kvq_torch as T

    B, Hq, Hkv, D, G = w["B"], w["Hq"], w["Hkv"], w["D"], w["G"]
    n = attended - 1  # cached rows before the step's append
    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[w["dtype"]]
    caches, steps_in = [], []
    for layer in layers:
        kp, ks, vp, vs = (layer[k][:, :, :n].cpu().contiguous() for k in ("kp", "ks", "vp", "vs"))
        caches.append(T.LayerCache(kp, ks, vp, vs, G))
        steps_in.append((layer["q"].cpu(), layer["knew"].cpu(), layer["vnew"].cpu()))
    scale = D ** -0.5
    threads = torch.get_num_threads()
    T.decode_step(caches[0], *steps_in[0], scale)  # warm up the operators once
    done, t0 = 0, time.perf_counter()
    while True:
        i = done % len(caches)
        c = caches[i]
        if c.kp.shape[2] > n + 64:  # keep each layer near the workload's context
            c.kp, c.ks, c.vp, c.vs = c.kp[:, :, :n].clone(), c.ks[:, :, :n].clone(), c.vp[:, :, :n].clone(), c.vs[:, :, :n].clone()
        T.decode_step(c, *steps_in[i], scale)
        done += 1
        if time.perf_counter() - t0 > budget_s and done >= max(2, len(caches)):  # every layer at least once
            break
    dt = time.perf_counter() - t0
    kv_tokens = int((seq_lens + 1).sum()) if seq_lens is not None else B * attended
    per = attn_bytes(w, kv_tokens) + append_bytes(w)

    # the C restatement on a shorter sample of the same layers
    c_threads = R.num_threads()
    sdt = "bf16" if w["dtype"] == "bf16" else "f16"
    sl = None if seq_lens is None else (seq_lens + 1).cpu().numpy()
    c_done, c_t0, c_budget = 0, time.perf_counter(), max(1.0, budget_s / 4)
    while True:
        c = caches[c_done % len(caches)]
        q, kn, vn = (x.float().numpy() for x in steps_in[c_done % len(caches)])
        R.quantize_int4(kn, G, sdt)
        R.quantize_int4(vn, G, sdt)
        R.decode_attn(q, c.kp.numpy(), c.ks.float().numpy(), c.vp.numpy(), c.vs.float().numpy(), group_size=G,
                      scale=scale, seq_lens=sl, threads=c_threads)
        c_done += 1
        if time.perf_counter() - c_t0 > c_budget and c_done >= 2:
            break
    c_dt = time.perf_counter() - c_t0
    return {
        "value": round(done * per / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done} layer-steps of {w['desc']} over its {len(caches)} layers (each its own cache, "
                  f"{len(caches) * per / 2**20:.0f} MiB), the reference's torch CPU path (quantize, torch.cat "
                  f"append, dequantize, repeat_interleave + SDPA; oracle/kvq_torch.py), {threads} torch threads, "
                  f"{dt:.1f} s",
        "ms_per_layer": round(dt / done * 1e3, 3),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "c_port": {"value": round(c_done * per / c_dt / 1e9, 3), "unit": "GB/s", "cores": c_threads,
                   "ms_per_layer": round(c_dt / c_done * 1e3, 3),
                   "sample": f"{c_done} layer-steps, oracle/kvq_ref.c (OpenMP, no concatenation), {c_dt:.1f} s"},
    }


if __name__ == "__main__":
    sys.exit(main())
