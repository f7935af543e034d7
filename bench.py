"""Headline benchmark: batch-1 routed-MoE expert GEMV on one MI355X.

Workload (config 3): 256 experts, hidden 2048, expert intermediate 512, top-8,
2-bit (K=2) coded gate_up and down per expert, hash decode.  L=40 independent
layer stacks (40 x 201,326,592 coded bytes = 8.05 GB, far above the 256 MB
Infinity Cache), so every routed expert is read cold from HBM.  Router logits
are seeded float32 N(0,1) per layer, routed top-8 with softmax weights.

One step = one token through the routed-expert path of all 40 layers,
chained (layer l's output is layer l+1's input), i.e. one decode step of the
MoE layers.  Inputs are resident in HBM before timing starts.

Reported: coded-weight GB/s (6,291,456 B per token-layer), decode tok/s,
roofline of the expert-path launch, and the NumPy oracle timed on the host
(cpu_baseline) on a bounded sample of the same work.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers 40] [--lut 0|1]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

E, H, I, TOP_K, K = 256, 2048, 512, 8, 2
BYTES_GU = H * 2 * I * K // 8          # 524,288 per expert
BYTES_DN = I * H * K // 8              # 262,144 per expert
BYTES_TOKEN_LAYER = TOP_K * (BYTES_GU + BYTES_DN)   # 6,291,456
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--lut", type=int, default=0)
    ap.add_argument("--cpu-sample", type=int, default=3, help="token-layers for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    return ap.parse_args()


def make_layers(torch, n_layers: int, dev: str, seed: int = 2):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        gu = torch.randint(-2**31, 2**31 - 1, (E, H // 16, 2 * I // 16, 8 * K), generator=g,
                           device=dev, dtype=torch.int32)
        dn = torch.randint(-2**31, 2**31 - 1, (E, I // 16, H // 16, 8 * K), generator=g,
                           device=dev, dtype=torch.int32)
        sgn = lambda *s: torch.where(torch.rand(*s, generator=g, device=dev) < 0.5, -1.0, 1.0)
        gu_rin, dn_rin = sgn(E, H), sgn(E, I)
        gu_rout = sgn(E, 2 * I) * (0.5 + torch.rand(E, 2 * I, generator=g, device=dev)) * 4e-2
        dn_rout = sgn(E, H) * (0.5 + torch.rand(E, H, generator=g, device=dev)) * 4e-2
        logits = torch.randn(1, E, generator=g, device=dev, dtype=torch.float32)
        layers.append(dict(gu=gu, dn=dn, gu_rin=gu_rin.float().contiguous(),
                           dn_rin=dn_rin.float().contiguous(), gu_rout=gu_rout.float().contiguous(),
                           dn_rout=dn_rout.float().contiguous(), logits=logits))
    return layers


def cpu_baseline(layers_np, n_sample: int):
    """The NumPy oracle (decode + transforms + f32 matmul, no weight cache), one BLAS thread."""
    from threadpoolctl import threadpool_limits

    from oracle import ref_np
    t_total = 0.0
    with threadpool_limits(limits=1):
        for s in range(n_sample):
            L = layers_np[s % len(layers_np)]
            x = L["x"]
            t0 = time.perf_counter()
            w_gu = {e: ref_np.reconstruct(L["gu"][e], H, 2 * I, K) for e in L["ids"][0]}
            w_dn = {e: ref_np.reconstruct(L["dn"][e], I, H, K) for e in L["ids"][0]}
            gu = {"w": w_gu, "rin": L["gu_rin"], "rout": L["gu_rout"]}
            dn = {"w": w_dn, "rin": L["dn_rin"], "rout": L["dn_rout"]}
            ref_np.moe_routed(x, L["ids"], L["scores"], gu, dn, K, K, ordered=False)
            t_total += time.perf_counter() - t0
    per = t_total / n_sample
    return {"value": round(BYTES_TOKEN_LAYER / per / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{n_sample} token-layers of config 3 through oracle/ref_np.py "
                      f"(vectorised decode of 8 experts x 2 legs, no cache, f32 matmul, 1 BLAS "
                      f"thread): {per * 1e3:.1f} ms per token-layer"}


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus N>1 is not supported "
                                   "(the coded-projection path shards per DESIGN.md but no "
                                   "multi-GPU run is part of this build)"}))
        sys.exit(2)
    import torch

    from escha_mlx_amd import moe, ops

    dev = "cuda:0"
    torch.cuda.set_device(0)
    ops.init()
    layers = make_layers(torch, args.layers, dev)
    ws = torch.zeros(ops.moe_expert_path_workspace(1, TOP_K, E, H, I), dtype=torch.uint8, device=dev)
    routes = [moe.route(L["logits"], TOP_K) for L in layers]
    x0 = torch.randn(1, H, generator=torch.Generator(device=dev).manual_seed(7), device=dev).half()
    outs = [torch.empty(1, H, dtype=torch.float16, device=dev) for _ in layers]
    stream = torch.cuda.current_stream()

    def step():
        x = x0
        for L, (ids, sc), y in zip(layers, routes, outs):
            ops.moe_expert_path(x, ids, sc, L["gu"], L["gu_rin"], L["gu_rout"], K, L["dn"],
                                L["dn_rin"], L["dn_rout"], K, lut=bool(args.lut), ws=ws, out=y)
            x = y
        return x

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = ev0.elapsed_time(ev1) / args.steps
    tok_s = 1e3 / ms
    gbs = BYTES_TOKEN_LAYER * args.layers / (ms * 1e-3) / 1e9
    launch_us = ms * 1e3 / args.layers

    result = {
        "metric": "coded-weight HBM GB/s (% of peak) + decode tok/s, 2-bit MoE GEMV at batch 1",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 codes -> f16 weights, f32 accumulate",
        "data": "synthetic: uniform-random code streams, seeded rin/rout/logits/x",
        "config": {"workload": "config 3: routed MoE expert GEMV, batch 1, E=256, H=2048, "
                               "I=512, top-8, K=2 gate_up+down, hash decode, 40 cold layers "
                               "chained per step",
                   "layers": args.layers, "bytes_per_token_layer": BYTES_TOKEN_LAYER,
                   "lut": args.lut},
        "tok_s": round(tok_s, 2),
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "launch": "esc_moe_expert_path (one token-layer)",
                     "avg_launch_us": round(launch_us, 3)},
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu:
        sample = []
        for li in range(min(args.cpu_sample, args.layers)):
            L = layers[li]
            ids, sc = routes[li]
            sample.append({
                "gu": L["gu"].cpu().numpy().view(np.uint32), "dn": L["dn"].cpu().numpy().view(np.uint32),
                "gu_rin": L["gu_rin"].cpu().numpy(), "dn_rin": L["dn_rin"].cpu().numpy(),
                "gu_rout": L["gu_rout"].cpu().numpy(), "dn_rout": L["dn_rout"].cpu().numpy(),
                "ids": ids.cpu().numpy(), "scores": sc.cpu().numpy(),
                "x": x0.cpu().numpy()})
        result["cpu_baseline"] = cpu_baseline(sample, args.cpu_sample)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
