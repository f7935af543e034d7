"""Headline benchmark: batch-1 routed-MoE expert GEMV on one MI355X.

Workload (config 3): 256 experts, hidden 2048, expert intermediate 512, top-8,
2-bit (K=2) coded gate_up and down per expert, hash decode.  L=40 independent
layer stacks (40 x 201,326,592 coded bytes = 8.05 GB, far above the 256 MB
Infinity Cache), so every routed expert is read cold from HBM.  Router logits
are seeded float32 N(0,1) per layer, routed top-8 with softmax weights.

Two measurements, both one token per layer (batch 1):
  sustained (the `value`): the 40 token-layers are independent and go to the
      GPU as ONE launch of esc_moe_expert_path_layers; steady-state coded-weight
      throughput of the expert GEMV (the protocol "sustained, back-to-back over
      independent layers").
  chained (`tok_s`): a decode step — layer l's output is layer l+1's input —
      as 40 launches of the drop-in esc_moe_expert_path; tok/s = 1 / step.
Inputs are resident in HBM before timing starts; HIP events on the launch stream.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers 40]
"""
from __future__ import annotations

import argparse
import json
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
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=40)
    ap.add_argument("--cpu-sample", type=int, default=3, help="token-layers for the CPU baseline")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", choices=["both", "sustained", "chained"], default="both")
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
        x = torch.randn(1, H, generator=g, device=dev).half()
        layers.append(dict(gu_code=gu, dn_code=dn, gu_rin=gu_rin.float().contiguous(),
                           dn_rin=dn_rin.float().contiguous(), gu_rout=gu_rout.float().contiguous(),
                           dn_rout=dn_rout.float().contiguous(), logits=logits, x=x))
    return layers


def cpu_baseline(sample, n_sample: int):
    """The NumPy oracle (decode + transforms + f32 matmul, no weight cache), one BLAS thread."""
    from threadpoolctl import threadpool_limits

    from oracle import ref_np
    t_total = 0.0
    with threadpool_limits(limits=1):
        for s in range(n_sample):
            L = sample[s % len(sample)]
            t0 = time.perf_counter()
            w_gu = {e: ref_np.reconstruct(L["gu"][e], H, 2 * I, K) for e in L["ids"][0]}
            w_dn = {e: ref_np.reconstruct(L["dn"][e], I, H, K) for e in L["ids"][0]}
            gu = {"w": w_gu, "rin": L["gu_rin"], "rout": L["gu_rout"]}
            dn = {"w": w_dn, "rin": L["dn_rin"], "rout": L["dn_rout"]}
            ref_np.moe_routed(L["x"], L["ids"], L["scores"], gu, dn, K, K, ordered=False)
            t_total += time.perf_counter() - t0
    per = t_total / n_sample
    return {"value": round(BYTES_TOKEN_LAYER / per / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"{n_sample} token-layers of config 3 through oracle/ref_np.py "
                      f"(vectorised decode of 8 experts x 2 legs, no cache, f32 matmul, 1 BLAS "
                      f"thread): {per * 1e3:.1f} ms per token-layer"}


def timed(torch, fn, steps: int, warmup: int, stream) -> float:
    """Average ms per call of fn(), HIP events on `stream` around `steps` calls."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for _ in range(steps):
        fn()
    ev1.record(stream)
    torch.cuda.synchronize()
    return ev0.elapsed_time(ev1) / steps


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus N>1 is not supported "
                                   "(DESIGN.md describes how the path would shard)"}))
        sys.exit(2)
    import torch

    from escha_mlx_amd import moe, ops

    dev = "cuda:0"
    torch.cuda.set_device(0)
    ops.init()
    nl = args.layers
    layers = make_layers(torch, nl, dev)
    for L in layers:
        L["ids"], L["scores"] = moe.route(L["logits"], TOP_K)
        L["y"] = torch.empty(1, H, dtype=torch.float16, device=dev)
    stream = torch.cuda.current_stream()
    t_wall = time.perf_counter()
    result = {
        "metric": "coded-weight HBM GB/s (% of peak) + decode tok/s, 2-bit MoE GEMV at batch 1",
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 codes -> f16 weights (hash decode), f32 accumulate",
        "data": "synthetic: uniform-random code streams, seeded rin/rout/logits/x (random-init)",
        "config": {"workload": "config 3: routed MoE expert GEMV, batch 1 per layer, E=256, "
                               "H=2048, I=512, top-8, K=2 gate_up+down, hash decode, "
                               f"{nl} cold layer stacks",
                   "layers": nl, "bytes_per_token_layer": BYTES_TOKEN_LAYER},
    }

    if args.only in ("both", "sustained"):
        table = ops.moe_layers_table(layers, dev)
        ws_l = torch.zeros(ops.moe_layers_workspace(nl, 1, TOP_K, H, I), dtype=torch.uint8,
                           device=dev)
        ms = timed(torch, lambda: ops.moe_expert_path_layers(table, 1, TOP_K, E, H, I, K, K,
                                                             ws=ws_l), args.steps, args.warmup,
                   stream)
        gbs = BYTES_TOKEN_LAYER * nl / (ms * 1e-3) / 1e9
        result.update({
            "value": round(gbs, 2),
            "ms_per_step": round(ms, 4),
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
            "sustained_us_per_token_layer": round(ms * 1e3 / nl, 3),
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "kernel": "k_moe_fused<2,2,16,32,false> (esc_moe_expert_path_layers)",
                         "bytes_per_launch": BYTES_TOKEN_LAYER * nl,
                         "avg_launch_us": round(ms * 1e3, 2)},
        })

    if args.only in ("both", "chained"):
        ws = torch.zeros(ops.moe_expert_path_workspace(1, TOP_K, E, H, I), dtype=torch.uint8,
                         device=dev)
        x0 = layers[0]["x"]

        def chained():
            x = x0
            for L in layers:
                ops.moe_expert_path(x, L["ids"], L["scores"], L["gu_code"], L["gu_rin"],
                                    L["gu_rout"], K, L["dn_code"], L["dn_rin"], L["dn_rout"], K,
                                    ws=ws, out=L["y"])
                x = L["y"]

        ms_c = timed(torch, chained, args.steps, args.warmup, stream)
        gbs_c = BYTES_TOKEN_LAYER * nl / (ms_c * 1e-3) / 1e9
        result.update({
            "tok_s": round(1e3 / ms_c, 2),
            "chained_ms_per_token": round(ms_c, 4),
            "chained_us_per_token_layer": round(ms_c * 1e3 / nl, 3),
            "chained_gbs": round(gbs_c, 2),
        })
        if "value" not in result:
            result.update({"value": round(gbs_c, 2), "ms_per_step": round(ms_c, 4)})
    result["wall_s"] = round(time.perf_counter() - t_wall, 3)

    if not args.no_cpu:
        sample = []
        for L in layers[: min(args.cpu_sample, nl)]:
            sample.append({
                "gu": L["gu_code"].cpu().numpy().view(np.uint32),
                "dn": L["dn_code"].cpu().numpy().view(np.uint32),
                "gu_rin": L["gu_rin"].cpu().numpy(), "dn_rin": L["dn_rin"].cpu().numpy(),
                "gu_rout": L["gu_rout"].cpu().numpy(), "dn_rout": L["dn_rout"].cpu().numpy(),
                "ids": L["ids"].cpu().numpy(), "scores": L["scores"].cpu().numpy(),
                "x": L["x"].cpu().numpy()})
        result["cpu_baseline"] = cpu_baseline(sample, args.cpu_sample)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
