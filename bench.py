"""Benchmark: one Qwen3-30B-A3B MoE layer at decode batch 1.

metric: us per MoE layer + achieved HBM GB/s (% of peak), 4-bit top-8, batch 1.
A step is one MoE layer: kernel 1 (gate_up+SiLU over the 8 routed experts) and
kernel 2 (down + routing-weighted sum), reading 4-bit group-128 experts from a
GPU slot pool. Routing is drawn per step (router logits ~ N(0,1) -> softmax ->
top-8 -> renormalise -> bf16), x ~ N(0,1) bf16, experts quantized from
N(0, 0.02) weights on the GPU. To measure HBM and not the 256 MB Infinity Cache,
steps rotate over 48 distinct layer pools of 128 experts (15.4 GB); the layer
sequence is captured once in a HIP graph and replayed (inputs resident in HBM).

`value` is algorithmic bytes per layer / time per layer (GB/s); `ms_per_step`
is the time per layer. The roofline object is for the dominant kernel
(kernel 1), timed with HIP events around graph replays of that kernel alone on
its own stream. The cpu_baseline is the reference's dequantize-then-matmul path
restated in torch and timed on this host's cores over a bounded sample.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "wisp-runtime_amd"))

import torch  # noqa: E402

from wisp import _lib  # noqa: E402
from wisp.moe import pack_meta, route  # noqa: E402
from wisp.quant import expert_nbytes, quantize  # noqa: E402

H, I, E, K_TOP, G = 2048, 768, 128, 8, 128
PEAK_HBM_GBS = 8000.0


def alg_bytes(bits: int):
    """Algorithmic HBM bytes of one layer, per kernel (codes + fp16 scales/mins of the
    k routed experts, x, the fp32-sized activation write/read, the meta reads, the output)."""
    n = H * I
    mat_codes = n * bits // 8
    mat_sm = 2 * 2 * (n // G)
    gu = K_TOP * 2 * (mat_codes + mat_sm) + 2 * H + 4 * K_TOP * I + 8 * K_TOP
    dn = K_TOP * (mat_codes + mat_sm) + 4 * K_TOP * I + 2 * H + 8 * K_TOP
    return gu, dn


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=960, help="timed MoE layers (rounded up to whole graph replays)")
    ap.add_argument("--warmup", type=int, default=96, help="untimed MoE layers")
    ap.add_argument("--bits", type=int, default=4, choices=[4, 3, 2])
    ap.add_argument("--layers", type=int, default=48, help="distinct layer pools rotated (>= 2 to defeat the MALL)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0, help="seconds of CPU baseline sampling")
    ap.add_argument("--tune", default="", help="gu_rows,gu_waves,dn_iters")
    a = ap.parse_args()

    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (single-GPU path; see DESIGN.md for how it would shard). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    L = _lib.lib()
    if a.tune:
        gr, gw, dn = (int(v) for v in a.tune.split(","))
        _lib.check(L.wisp_set_tuning(gr, gw, dn), "set_tuning")

    bits, layers = a.bits, a.layers
    n = H * I
    nb = expert_nbytes(n, bits, G)
    print(f"[bench] quantizing {E} experts ({bits}-bit, {nb} B each) on the GPU", file=sys.stderr, flush=True)
    gen = torch.Generator(device=dev).manual_seed(2)
    base = torch.empty((E, nb), dtype=torch.uint8, device=dev)
    for e in range(E):
        w3 = torch.randn((3, n), generator=gen, device=dev) * 0.02
        base[e].copy_(quantize(w3, bits, G))
    pool = torch.empty((layers * E, nb), dtype=torch.uint8, device=dev)
    for l in range(layers):
        pool[l * E : (l + 1) * E].copy_(base)
    del base
    torch.cuda.synchronize()
    print(f"[bench] slot pool {pool.numel() / 2**30:.2f} GiB ({layers} layers x {E} experts)", file=sys.stderr,
          flush=True)

    # routing and inputs for `rounds` distinct replays of the layer sequence
    rounds = 8
    g2 = torch.Generator(device=dev).manual_seed(3)
    logits = torch.randn((rounds, layers, E), generator=g2, device=dev)
    sel, rw = route(logits.reshape(-1, E), K_TOP)
    slots = sel.reshape(rounds, layers, K_TOP) + (torch.arange(layers, device=dev) * E).view(1, layers, 1)
    metas = pack_meta(slots, rw.reshape(rounds, layers, K_TOP)).contiguous()  # [rounds, layers, 2k]
    xs = (torch.randn((layers, H), generator=g2, device=dev)).to(torch.bfloat16)
    meta_live = torch.empty((layers, 2 * K_TOP), dtype=torch.float32, device=dev)
    meta_live.copy_(metas[0])
    act = torch.empty((layers, K_TOP, I), dtype=torch.int32, device=dev)
    out = torch.empty((layers, H), dtype=torch.bfloat16, device=dev)

    stream = torch.cuda.Stream(dev)
    sp = _lib.ptr

    def gate_up(l, st):
        _lib.check(L.wisp_moe_gate_up(sp(pool), nb, pool.shape[0], sp(meta_live[l]), K_TOP, sp(xs[l]), H, I, bits,
                                      G, sp(act[l]), st), "gate_up")

    def down(l, st):
        _lib.check(L.wisp_moe_down_sum(sp(pool), nb, pool.shape[0], sp(meta_live[l]), K_TOP, sp(act[l]), H, I,
                                       bits, G, sp(out[l]), st), "down_sum")

    def capture(body):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            st = _lib.stream(dev)
            for l in range(layers):  # eager warm-up of the same launches
                body(l, st)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=stream):
                st = _lib.stream(dev)
                for l in range(layers):
                    body(l, st)
        torch.cuda.synchronize()
        return g

    g_layer = capture(lambda l, st: (gate_up(l, st), down(l, st)))
    g_gu = capture(gate_up)
    g_dn = capture(down)

    def run(g, reps, swap_meta):
        with torch.cuda.stream(stream):
            for r in range(reps):
                if swap_meta:
                    meta_live.copy_(metas[r % rounds], non_blocking=True)
                g.replay()

    def timed(g, reps, swap_meta):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        run(g, reps, swap_meta)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3  # seconds

    warm_reps = max(1, -(-a.warmup // layers))
    reps = max(1, -(-a.steps // layers))
    steps = reps * layers
    print(f"[bench] warm-up {warm_reps * layers} layers, timing {steps} layers", file=sys.stderr, flush=True)
    run(g_layer, warm_reps, True)
    torch.cuda.synchronize()
    t_layer = timed(g_layer, reps, True)
    t_gu = timed(g_gu, reps, False)
    t_dn = timed(g_dn, reps, False)

    gu_b, dn_b = alg_bytes(bits)
    layer_b = gu_b + dn_b
    s_layer = t_layer / steps
    s_gu = t_gu / steps
    s_dn = t_dn / steps
    value = layer_b / s_layer / 1e9
    ach_gu = gu_b / s_gu / 1e9

    res = {
        "metric": "us per MoE layer + achieved HBM GB/s (% of peak), 4-bit top-8, batch 1"
        if bits == 4 else f"us per MoE layer + achieved HBM GB/s (% of peak), {bits}-bit top-8, batch 1",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warm_reps * layers,
        "ms_per_step": round(s_layer * 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic",
        "config": {
            "workload": f"C2: one Qwen3-30B-A3B MoE layer, decode batch 1, top-{K_TOP} of {E} experts, {bits}-bit "
                        f"group-{G}, H={H} I={I}, {layers} layer pools rotated",
            "weights": f"u{bits} group-{G} fp16 scale+min",
            "accumulate": "fp32 (bf16 x dot2)",
            "bytes_per_layer": layer_b,
        },
        "us_per_layer": round(s_layer * 1e6, 3),
        "pct_hbm_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "kernels": {
            "gate_up_us": round(s_gu * 1e6, 3),
            "down_us": round(s_dn * 1e6, 3),
            "sum_us": round((s_gu + s_dn) * 1e6, 3),
            "gate_up_bytes": gu_b,
            "down_bytes": dn_b,
            "gate_up_GBs": round(ach_gu, 1),
            "down_GBs": round(dn_b / s_dn / 1e9, 1),
            "timing": "HIP events around graph replays of each kernel alone (per-launch average, incl. "
                      "in-graph launch gaps)",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(ach_gu, 1),
            "peak": PEAK_HBM_GBS,
            "unit": "GB/s",
            "frac": round(ach_gu / PEAK_HBM_GBS, 4),
            "traffic": None,
        },
        "cpu_baseline": None,
    }

    if not a.no_cpu_baseline:
        sys.path.insert(0, ROOT)
        from oracle import cpu_baseline as CB  # the checker/baseline side only

        # bounded sample: 96 distinct experts from one layer pool on the host, 8 routed per layer
        rows = pool[:96].cpu()
        routes = []
        lg = torch.randn((64, 96), generator=torch.Generator().manual_seed(5))
        s_cpu, w_cpu = route(lg, K_TOP)
        routes = [(s_cpu[i].tolist(), w_cpu[i].float().tolist()) for i in range(64)]
        xcpu = [xs[i % layers].cpu() for i in range(8)]
        med, cnt, thr = CB.time_layers(rows, routes, xcpu, H, I, bits, G, budget_s=a.cpu_budget)
        res["cpu_baseline"] = {
            "value": round(layer_b / med / 1e9, 3),
            "unit": "GB/s",
            "cores": thr,
            "kind": "port",
            "sample": f"{cnt} MoE layers (8 of 96 distinct experts each, rotated), median; torch dequant->bf16 "
                      f"F.linear on {thr} threads; {round(med * 1e6, 1)} us/layer; cpu={platform.processor() or 'x86_64'}",
            "us_per_layer": round(med * 1e6, 1),
        }
    print(json.dumps(res))


if __name__ == "__main__":
    main()
