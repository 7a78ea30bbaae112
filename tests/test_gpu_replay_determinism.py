"""GPU: determinism of the north-star decode step under graph replay. The
step (Llama-3.1-8B attention shape: 32 query / 8 KV heads, head dim 128,
group 32, 16,384 cached keys; 32 layers, each its own INT4 cache and one
fused decode-step launch) is captured in one HIP graph and replayed 1000
times. Each replay rewrites the same new row, re-arms the split counters and
reuses the workspace, so every replay's 32 outputs must equal the first
replay's bit for bit: the split merge combines the partials in a fixed
order, whichever workgroup arrives last. Stops at the first mismatch."""

from __future__ import annotations

import pytest
import torch

from kvint4 import ops

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def test_ns_step_graph_1000_replays_bit_identical():
    B, Hq, Hkv, D, G, ctx, L = 1, 32, 8, 128, 32, 16384, 32
    g = torch.Generator(device=DEV).manual_seed(21)
    W, NG = ops.packed_width(D, G), ops.num_groups(D, G)
    stream = torch.cuda.Stream(DEV)
    layers = []
    outs = torch.empty(L, B, Hq, 1, D, dtype=torch.bfloat16, device=DEV)
    with torch.cuda.stream(stream):
        for _ in range(L):
            lay = {}
            for name in ("k", "v"):
                packed = torch.empty(B, Hkv, ctx + 1, W, dtype=torch.uint8, device=DEV)
                scales = torch.empty(B, Hkv, ctx + 1, NG, dtype=torch.bfloat16, device=DEV)
                x = torch.randn(B, Hkv, ctx, D, generator=g, device=DEV).to(torch.bfloat16)
                ops.quantize_into(x, packed, scales, G, 0)
                lay[name + "p"], lay[name + "s"] = packed, scales
            for name, h in (("q", Hq), ("kn", Hkv), ("vn", Hkv)):
                lay[name] = torch.randn(B, h, 1, D, generator=g, device=DEV).to(torch.bfloat16)
            layers.append(lay)
    torch.cuda.synchronize()

    def step():
        for i, lay in enumerate(layers):
            ops.decode_step(lay["q"], lay["kn"], lay["vn"], lay["kp"], lay["ks"], lay["vp"], lay["vs"], ctx,
                            n_kv_heads=Hkv, group_size=G, sm_scale=D ** -0.5, out=outs[i])

    with torch.cuda.stream(stream):
        step()  # warm-up: allocates the workspace outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        step()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        graph.replay()
    torch.cuda.synchronize()
    first = outs.clone()
    assert torch.isfinite(first.float()).all()
    for r in range(1, 1000):
        with torch.cuda.stream(stream):
            graph.replay()
        torch.cuda.synchronize()
        if not torch.equal(outs, first):
            bad = [i for i in range(L) if not torch.equal(outs[i], first[i])]
            pytest.fail(f"replay {r}: layers {bad} differ from the first replay")
    print("NS step graph: 1000 replays, every output bit-identical to the first", flush=True)
