"""Benchmark: hot/cold sparse-FFN decode on one MI355X.

Workload (one "step" = one token through the stack): 32 FFN layers of
4096 x 14336 SwiGLU, batch 1, the residual stream carried between layers with
RMSNorm in front of every FFN; 25 % of each layer's neurons hot (fp8 e4m3 with
per-row fp32 scales, resident in HBM), the rest cold INT4 records in the split
format, resident in HBM; a random-init bf16 predictor per layer
(4096 -> 64 -> 14336) with its threshold calibrated so ~5 % of neurons are
predicted active, selecting layer L+1's cold neurons from layer L's input.
Weights are N(0, 0.02) from a fixed seed (synthetic data, nothing loaded).

Prints one JSON line.  `value` is tokens/s with every input already in HBM.
`roofline` is the ffn_up kernel (hot gate/up + cold gather/dequant/act/down +
lookahead predictor projection), timed per launch with hipEvents on its
stream; `cpu_baseline` is the restated reference CPU path (per-neuron
record decode loop + F.linear FFN) on a bounded sample of the same token.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "hot-cold-neural-split-openinfer2_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

H, INTER, N_LAYERS, N_HOT, RANK = 4096, 14336, 32, 3584, 64
ACTIVE_FRAC = 0.05
EPS = 1e-5
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_stack(seed, dev):
    import torch
    from oi2.stack import DecodeStack, StackLayer
    from oi2.synth import SyntheticLayer, calibrate_threshold
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = []
    for i in range(N_LAYERS):
        layers.append(SyntheticLayer(g, INTER, N_HOT, std=0.02, device=dev, with_predictor=True,
                                     pred_rank=RANK, pred_dtype=torch.bfloat16))
    thr = calibrate_threshold(layers, g, ACTIVE_FRAC)
    st = DecodeStack([StackLayer(l.hot, l.records, l.lut, l.norm_w, l.predictor) for l in layers],
                     INTER, EPS, "silu", False, thr)
    # size the cold pass for the calibrated active fraction with headroom
    st.set_expected_active(int(1.3 * ACTIVE_FRAC * (INTER - N_HOT)))
    return layers, st, thr, g


def up_launch_bytes(active):
    """Algorithmic bytes of one ffn_up launch: hot gate+up fp8 rows and their
    scales, every active cold record (6400 B), the lookahead predictor's bf16
    down projection, the token, two norm weights, and the h/z writes."""
    return (2 * N_HOT * H + 2 * N_HOT * 4 + active * 6400 + RANK * H * 2 + 3 * H * 2
            + N_HOT * 4 + RANK * 4)


def down_launch_bytes(active_next):
    """ffn_down: hot down fp8 rows + row scales, h_hot, the predictor's bf16 up
    projection + bias, the LUT, x in/out, and the compacted selection."""
    return (H * N_HOT + H * 4 + N_HOT * 4 + INTER * RANK * 2 + INTER * 2 + INTER * 4
            + 2 * H * 2 + active_next * 8)


def cpu_baseline(layers, xs_in, active_ids, n_sample, dev):
    """Restated reference CPU path over the first n_sample layers of one token."""
    import numpy as np
    import torch
    from oracle import baseline_cpu as B
    samples = []
    for L in range(n_sample):
        lay = layers[L]
        recs = lay.records.cpu().numpy()
        buf = memoryview(recs.reshape(-1))
        nids = lay.cold_ids.cpu().numpy()
        offs = {int(n): int(k) * 6400 for k, n in enumerate(nids)}
        hot = lay.hot
        gate = (hot.gate_q.view(torch.float8_e4m3fn).float() * hot.gate_scale[:, None]).cpu()
        up = (hot.up_q.view(torch.float8_e4m3fn).float() * hot.up_scale[:, None]).cpu()
        down = (hot.down_q[:, :hot.n_hot].contiguous().view(torch.float8_e4m3fn).float()
                * hot.down_scale[:, None]).cpu()
        x = xs_in[L].float().cpu()[None]
        xn = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + EPS) * lay.norm_w.float().cpu()
        samples.append((xn, (gate, up, down), buf, offs, active_ids[L]))
    secs, neurons, nbytes = B.time_layers(samples, threads=1)
    per_layer = secs / n_sample
    return {
        "value": 1.0 / (per_layer * N_LAYERS),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "sample": (f"{n_sample} of 32 layers of one token ({neurons} cold neurons, "
                   f"{nbytes / 1e6:.1f} MB of records) through the restated reference CPU path "
                   f"(per-neuron bytes/frombuffer/dequantize_int4 loop + fp32 F.linear FFN), "
                   f"1 torch thread, {secs:.1f} s; scaled to 32 layers"),
        "cold_neurons_per_s": neurons / secs,
        "seconds": secs,
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--profile-tokens", type=int, default=8)
    ap.add_argument("--cpu-sample-layers", type=int, default=16)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import oi2  # noqa: F401
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    t0 = time.time()
    layers, st, thr, g = build_stack(args.seed, dev)
    torch.cuda.synchronize()
    log(f"built 32-layer stack in {time.time() - t0:.1f}s, threshold logit {thr:.4f}")

    stream = torch.cuda.Stream(device=dev)
    bufs = [torch.randn(H, generator=g, device=dev).half(), torch.empty(H, dtype=torch.float16, device=dev)]
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            st.decode(bufs[i % 2], bufs[(i + 1) % 2], stream)
    stream.synchronize()
    torch.cuda.synchronize()
    log(f"warmup {args.warmup} tokens done")

    base = args.warmup
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    with torch.cuda.stream(stream):
        ev0.record(stream)
        for i in range(args.steps):
            k = base + i
            st.decode(bufs[k % 2], bufs[(k + 1) % 2], stream)
        ev1.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    gpu_ms = ev0.elapsed_time(ev1)
    secs = max(wall, gpu_ms / 1e3)
    tok_s = args.steps / secs
    log(f"timed {args.steps} tokens: {secs * 1e3:.2f} ms ({tok_s:.1f} tok/s)")

    # per-launch kernel timing with hipEvents on the launch stream
    up_t, down_t, up_b, down_b, act_counts = [], [], [], [], []
    x_last_in = None
    k = base + args.steps
    for p in range(args.profile_tokens):
        xi, xo = bufs[(k + p) % 2], bufs[(k + p + 1) % 2]
        x_last_in = xi.clone()
        with torch.cuda.stream(stream):
            u, d = st.profile(xi, xo, stream)
        xs, counts, slots, ids = st.trace()
        torch.cuda.synchronize()
        c = counts.sum(1).cpu().tolist()
        act_counts.append(c)
        for L in range(N_LAYERS):
            up_t.append(u[L])
            down_t.append(d[L])
            up_b.append(up_launch_bytes(c[L]))
            down_b.append(down_launch_bytes(c[L + 1] if L + 1 < N_LAYERS else 0))
    up_ms = sum(up_t) / len(up_t)
    down_ms = sum(down_t) / len(down_t)
    up_gbs = sum(up_b) / (sum(up_t) / 1e3) / 1e9
    down_gbs = sum(down_b) / (sum(down_t) / 1e3) / 1e9
    mean_active = sum(sum(c) for c in act_counts) / (len(act_counts) * N_LAYERS)
    token_bytes = sum(up_b) / args.profile_tokens + sum(down_b) / args.profile_tokens
    log(f"ffn_up {up_ms * 1e3:.2f} us/launch {up_gbs:.0f} GB/s; ffn_down {down_ms * 1e3:.2f} us "
        f"{down_gbs:.0f} GB/s; mean active cold {mean_active:.0f}")

    cpu = None
    if not args.no_cpu_baseline and args.cpu_sample_layers > 0:
        xs, counts, slots, ids = st.trace()
        torch.cuda.synchronize()
        xs_in = [x_last_in] + [xs[i] for i in range(N_LAYERS - 1)]
        active = [st.active_ids(L, counts, ids) for L in range(N_LAYERS)]
        # cold ids -> the restated loop looks them up by neuron id
        n = min(args.cpu_sample_layers, N_LAYERS)
        cpu = cpu_baseline(layers, xs_in, active, n, dev)
        log(f"cpu baseline {cpu['value']:.4f} tok/s over {cpu['seconds']:.1f}s")

    out = {
        "metric": "FFN decode tok/s (32L, 4096x14336, bs1); cold INT4 dequant GB/s vs HBM",
        "value": tok_s,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": secs * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3+int4 weights, fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, random-init bf16 predictors)",
        "config": {"workload": "32-layer 4096x14336 SwiGLU hot/cold FFN decode, batch 1, 25% hot "
                               "fp8 in HBM, cold INT4 records in HBM, bf16 predictor at 5% active",
                   "layers": N_LAYERS, "hidden": H, "intermediate": INTER, "n_hot": N_HOT,
                   "batch": 1, "mean_active_cold": round(mean_active, 1),
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": up_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": up_gbs / HBM_PEAK_GBS, "traffic": None,
                     "kernel": "k_ffn_up", "us_per_launch": up_ms * 1e3,
                     "bytes_per_launch": sum(up_b) / len(up_b)},
        "kernels": {"k_ffn_down": {"us_per_launch": down_ms * 1e3, "achieved_gbs": down_gbs,
                                   "bytes_per_launch": sum(down_b) / len(down_b)}},
        "token_bytes": token_bytes,
        "hbm_frac_end_to_end": token_bytes * tok_s / (HBM_PEAK_GBS * 1e9),
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    st.close()


if __name__ == "__main__":
    main()
