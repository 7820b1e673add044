"""Benchmark: hot/cold sparse-FFN decode on one MI355X.

Workload (one "step" = one token through the stack): 32 FFN layers of
4096 x 14336 SwiGLU, batch 1, the residual stream carried between layers with
RMSNorm in front of every FFN; 25 % of each layer's neurons hot (fp8 e4m3 with
per-row fp32 scales, resident in HBM), the rest cold INT4 records in the split
format; a random-init bf16 predictor per layer (4096 -> 64 -> 14336) with its
threshold calibrated so ~5 % of neurons are predicted active, selecting layer
L+1's cold neurons from layer L's input.  Weights are N(0, 0.02) from a fixed
seed (synthetic data, nothing loaded).

Prints one JSON line.  `value` is tokens/s of that workload with the cold
store in pinned host memory and each layer's active records staged into HBM
over PCIe one layer ahead (a copy kernel on a side stream beside the FFN,
signalled on the device): the PCIe-bound configuration.  Every other input
(hot weights, predictors, the token) is already in HBM.  `staging` reports the
H2D rate against the measured link.  `hbm_resident` is the same workload with
the records in HBM too, decoded by the persistent token kernel; `roofline` is
that kernel (k_token), the decode path's dominant HBM kernel: its mean
duration from back-to-back launches between two hipEvents on the launch
stream, its algorithmic bytes the 32 layers' weights it must read (hot
gate/up/down fp8 rows and scales, every active cold record, both predictor
projections) plus the token and per-layer activations.  `cold_dequant` is the
fused cold INT4 gather/dequant/FFN kernel alone, and the read_neurons
dequant, in GB/s of records against the HBM peak.  `cpu_baseline` is the
restated reference CPU path (per-neuron record decode loop + F.linear FFN)
over a few recorded tokens, bounded to ~20 s.
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
# HBM bytes per launch on this workload, from rocprofv3 --pmc runs
# (FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 KiB, the factors being what each
# counter reads for a plain 256 MiB copy, --copy-calibration)
TOKEN_TRAFFIC_BYTES = (848467.9 * 2.0 + 115692.4) * 1024    # k_token
TOKEN_TRAFFIC_SOURCE = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of k_token on this workload, "
                        "profiles/k_token_traffic_decode32_bs1.md")
COPY_WORKGROUPS = 8          # the staging copy kernel's workgroups (swept: 6 / 8 / 10 / 12 / 16)
READER_THREADS = 8           # file store reader threads for batch 8 (8 and 16 measured alike)


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def build_stack(seed, dev):
    from oi2.synth import build_decode_stack
    return build_decode_stack(seed, dev, N_LAYERS, INTER, N_HOT, RANK, ACTIVE_FRAC, EPS)


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


def _hot_dense_cpu(hot):
    import torch
    gate = (hot.gate_q.view(torch.float8_e4m3fn).float() * hot.gate_scale[:, None]).cpu()
    up = (hot.up_q.view(torch.float8_e4m3fn).float() * hot.up_scale[:, None]).cpu()
    down = (hot.down_q[:, :hot.n_hot].contiguous().view(torch.float8_e4m3fn).float()
            * hot.down_scale[:, None]).cpu()
    return gate, up, down


def cpu_baseline(layers, tokens, max_seconds):
    """The restated reference CPU path (oracle.baseline_cpu) over the recorded
    tokens, layer by layer, until max_seconds of timed CPU work.

    tokens: list of (xs_in (32 fp16 layer inputs), active cold ids per layer)."""
    import numpy as np
    import torch
    from oracle import baseline_cpu as B
    secs = cold_secs = 0.0
    neurons = n_steps = 0
    calls, fetches, call_neurons = [], [], []
    for L in range(N_LAYERS):
        if secs >= max_seconds:
            break
        lay = layers[L]
        buf = memoryview(lay.records.cpu().numpy().reshape(-1))
        offs = {int(n): k * 6400 for k, n in enumerate(lay.cold_ids.cpu().tolist())}
        hot = _hot_dense_cpu(lay.hot)
        w = lay.norm_w.float().cpu()
        samples = []
        for xs_in, active in tokens:
            x = xs_in[L].float().cpu()[None]
            xn = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + EPS) * w
            samples.append((xn, hot, buf, offs, active[L]))
        dt, dc, nn, cl, fe = B.time_layers(samples, threads=1)
        calls += cl
        fetches += fe
        call_neurons += [len(a) for (_, _, _, _, a) in samples]
        secs += dt
        cold_secs += dc
        neurons += nn
        n_steps += len(samples)
    per_layer = secs / n_steps
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count()
    return {
        "value": 1.0 / (per_layer * N_LAYERS),
        "unit": "tok/s",
        "cores": 1,
        "kind": "port",
        "host_cpu_count": os.cpu_count(),
        "host_affinity_cpus": affinity,
        "torch_threads_default": torch.get_num_threads(),
        "sample": (f"{n_steps} layer-steps ({len(tokens)} tokens x {n_steps // len(tokens)} of 32 "
                   f"layers, {neurons} cold neurons) through the restated reference CPU path "
                   f"(per-neuron bytes/frombuffer/dequantize_int4 record loop + fp32 F.linear "
                   f"hot and cold FFN), 1 torch thread, {secs:.1f} s timed; scaled to 32 layers"),
        "seconds": secs,
        "cold_seconds": cold_secs,
        "cold_neurons_per_s": neurons / cold_secs,
        # per layer call (one layer of one token, the reference's FFN call),
        # the median over every timed call
        "layer_calls": len(calls),
        "median_layer_call_ms": float(np.median(calls)) * 1e3,
        "median_cold_fetch_ms": float(np.median(fetches)) * 1e3,
        "median_cold_neurons_per_call": float(np.median(call_neurons)),
        "median_call_cold_neurons_per_s": float(np.median(np.array(call_neurons) / np.array(fetches))),
    }


def timed_decode(st, x0, stream, warmup, steps):
    """Warm up, then time `steps` tokens back to back on `stream` (each fed
    the previous output) between two events, bracketed by synchronisation;
    status() after each phase raises if a device-side wait overran."""
    import torch
    bufs = [x0.clone(), torch.empty_like(x0)]
    with torch.cuda.stream(stream):
        for i in range(warmup):
            st.decode(bufs[i % 2], bufs[(i + 1) % 2], stream)
    stream.synchronize()
    st.status(stream)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t_start = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for i in range(steps):
            k = warmup + i
            st.decode(bufs[k % 2], bufs[(k + 1) % 2], stream)
        e1.record(stream)
    stream.synchronize()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_start
    st.status(stream)
    secs = max(wall, e0.elapsed_time(e1) / 1e3)
    k = warmup + steps
    return secs, bufs[k % 2]


def advance(st, x, stream, n):
    """The chain's input after n tokens from x."""
    import torch
    a, b = x.clone(), torch.empty_like(x)
    with torch.cuda.stream(stream):
        for _ in range(n):
            st.decode(a, b, stream)
            a, b = b, a
    stream.synchronize()
    st.status(stream)
    return a


def mean_active_over(st, x, stream, n):
    """Mean active cold records per layer over n tokens of the chain from x,
    and the chain's output after them."""
    import torch
    tot = 0.0
    a, b = x.clone(), torch.empty_like(x)
    for _ in range(n):
        with torch.cuda.stream(stream):
            st.decode(a, b, stream)
        stream.synchronize()
        _, counts, _, _ = st.trace()
        torch.cuda.synchronize()
        tot += counts.sum(1).float().mean().item()
        a, b = b, a
    st.status(stream)
    return tot / n, a


def pcie_link_gbs(dev):
    """The link reference: one 256 MiB pinned host -> device copy, 4 times."""
    import torch
    src = torch.empty(256 << 20, dtype=torch.uint8).pin_memory()
    dst = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    dst.copy_(src, non_blocking=True)
    torch.cuda.synchronize()
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record()
    for _ in range(4):
        dst.copy_(src, non_blocking=True)
    c1.record()
    torch.cuda.synchronize()
    gbs = 4 * src.numel() / (c0.elapsed_time(c1) / 1e3) / 1e9
    del src, dst
    return gbs


def build_staged(layers, thr):
    """The same 32 layers with every layer's cold records in pinned host
    memory, staged into HBM one layer ahead by COPY_WORKGROUPS copy
    workgroups."""
    import torch
    from oi2.stack import DecodeStack, StackLayer
    t0 = time.time()
    pinned = [l.records.cpu().pin_memory() for l in layers]
    sst = DecodeStack([StackLayer(l.hot, p, l.lut, l.norm_w, l.predictor)
                       for l, p in zip(layers, pinned)], INTER, EPS, "silu", False, thr,
                      staging=COPY_WORKGROUPS)
    sst.set_expected_active(int(1.3 * ACTIVE_FRAC * (INTER - N_HOT)))
    log(f"pinned host store {sum(p.numel() for p in pinned) / 1e9:.2f} GB in {time.time() - t0:.1f}s")
    return sst, pinned


def measure_token_phases(st, g, dev, tokens, warmup=16):
    """The persistent token kernel's phase timeline: `tokens` tokens traced
    after `warmup` plain ones (oi2_stack_trace_token: every group's control
    wave stamps eight points of each layer on the 100 MHz counter).  Per
    layer, over the groups: each step's median duration, the skew of the two
    arrivals (last group minus the median group) and the time from the last
    arrival to the median group seeing the signal; then the medians of those
    over the layers 1..30 and the tokens."""
    import numpy as np
    import torch
    stream = torch.cuda.Stream(device=dev)
    x0 = torch.randn(H, generator=g, device=dev).half()
    _, x = timed_decode(st, x0, stream, 0, warmup)
    steps = ["U inputs (U start -> B1)", "U products (B1 -> B2)", "U stores + arrival (B2 -> U arrival)",
             "U signal wait (U arrival -> U seen)", "D inputs (U seen -> D1a)", "D products + list (D1a -> D1b)",
             "D epilogue + arrival (D1b -> D arrival)", "D signal wait (D arrival -> next U start)"]
    per = {k: [] for k in steps}
    extra = {"layer_us": [], "u_arrival_skew_us": [], "u_signal_after_last_us": [],
             "d_arrival_skew_us": [], "d_signal_after_last_us": []}
    y = torch.empty_like(x)
    for _ in range(tokens):
        with torch.cuda.stream(stream):
            t = st.trace_token(x, y, stream)
        stream.synchronize()
        st.status(stream)
        a = t.cpu().numpy().astype(np.int64) / 100.0        # us, (L, 256, 8)
        x, y = y, x
        for L in range(1, a.shape[0] - 1):
            cur, nxt = a[L], a[L + 1]
            d = [cur[:, k + 1] - cur[:, k] for k in range(7)] + [nxt[:, 0] - cur[:, 7]]
            for k, name in enumerate(steps):
                per[name].append(float(np.median(d[k])))
            extra["layer_us"].append(float(np.median(nxt[:, 0] - cur[:, 0])))
            extra["u_arrival_skew_us"].append(float(cur[:, 3].max() - np.median(cur[:, 3])))
            extra["u_signal_after_last_us"].append(float(np.median(cur[:, 4]) - cur[:, 3].max()))
            extra["d_arrival_skew_us"].append(float(cur[:, 7].max() - np.median(cur[:, 7])))
            extra["d_signal_after_last_us"].append(float(np.median(nxt[:, 0]) - cur[:, 7].max()))
    out = {"tokens": tokens, "layers_summarised": "1..30", "unit": "us",
           "median_group_step": {k: float(np.median(v)) for k, v in per.items()}}
    out.update({k: float(np.median(v)) for k, v in extra.items()})
    for k, v in out["median_group_step"].items():
        log(f"token phases: {k:42s} {v:6.2f} us")
    for k in extra:
        log(f"token phases: {k:42s} {out[k]:6.2f} us")
    return out


def measure_cold_dequant(layers, dev, reps=4):
    """The cold INT4 path alone, in GB/s of records against the HBM peak.
    fused: oi2_ffn_forward with no hot half over every cold record of a layer
    (10752 records, 68.8 MB: the fetch-everything case of a layer without a
    predictor), all 32 layers back to back (1.05 GB of distinct records), so
    nothing is served from cache; the two launches per layer (gather,
    dequantise, gate/up dot, activation, down accumulate into partial rows;
    then the partial-row sum) are timed together.
    read_neurons: oi2_dequant_records on config 1's active set (1147 records)
    of each layer, fp32 gate/up/down out, as ColdWeightStore.read_neurons
    returns them."""
    import torch
    from oi2.layer import ColdNeurons, _ffn, workspace_bytes
    from oi2.store import ColdSection
    from oi2 import _lib
    x = torch.randn((1, H), device=dev).half()
    colds, wss = [], []
    for l in layers:
        n = l.records.shape[0]
        sec = ColdSection(0, l.cold_ids.cpu().numpy(), l.records, l.lut, l.lut.cpu().numpy(), INTER)
        c = ColdNeurons.from_slots(sec, torch.arange(n, dtype=torch.int32, device=dev))
        c.expected = 2048           # 512 cold workgroups, ~5 records per wave
        colds.append(c)
    ws = torch.empty(workspace_bytes(1, None, colds[0]), dtype=torch.uint8, device=dev)
    for l, c in zip(layers, colds):
        _ffn(x, l.norm_w, EPS, None, c, "silu", False, add_residual=True, workspace=ws)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        for l, c in zip(layers, colds):
            _ffn(x, l.norm_w, EPS, None, c, "silu", False, add_residual=True, workspace=ws)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    n_rec = layers[0].records.shape[0]
    rec_bytes = n_rec * 6400
    fused = {"records": n_rec, "us_per_layer": us, "record_gbs": rec_bytes / (us * 1e-6) / 1e9,
             "frac_of_hbm_peak": rec_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS,
             "neurons_per_s": n_rec / (us * 1e-6)}
    # read_neurons: dequantised fp32 tensors out
    L = _lib.lib()
    g = torch.Generator(device=dev).manual_seed(3)
    n_act = 1147
    slots = [torch.randperm(l.records.shape[0], generator=g, device=dev)[:n_act].int() for l in layers]
    outs = [torch.empty((n_act, H), dtype=torch.float32, device=dev) for _ in range(2)] + \
        [torch.empty((H, n_act), dtype=torch.float32, device=dev)]

    def dq(l, sl):
        _lib.check(L.oi2_dequant_records(l.records.data_ptr(), l.records.shape[0], sl.data_ptr(), n_act,
                                         outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
                                         _lib.stream_handle(dev)))
    for l, sl in zip(layers, slots):
        dq(l, sl)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(reps):
        for l, sl in zip(layers, slots):
            dq(l, sl)
    e1.record()
    torch.cuda.synchronize()
    us2 = e0.elapsed_time(e1) * 1e3 / (reps * len(layers))
    rb = n_act * 6400
    wb = 3 * n_act * H * 4
    read = {"records": n_act, "us": us2, "record_gbs": rb / (us2 * 1e-6) / 1e9,
            "hbm_gbs_records_plus_fp32_out": (rb + wb) / (us2 * 1e-6) / 1e9,
            "frac_of_hbm_peak": (rb + wb) / (us2 * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "neurons_per_s": n_act / (us2 * 1e-6)}
    return {"fused_cold_ffn": fused, "read_neurons_dequant": read}


def measure_batch8_file(dev, steps, warmup, seed=4):
    """Survey config 4: 32 layers, batch 8, Zipf(1.1) neuron popularity (hot =
    the top 20 % by rank, 2867 fp8 neurons), the cold records read from the
    page-aligned split file on every step (engine.py:266-290's fetch,
    splitter.py:354-403) into pinned buffers and moved to HBM with
    hipMemcpyAsync, each layer's set selected from the batch-mean query.
    Timed twice: through the mapping with the file in the page cache (warm),
    and with O_DIRECT page reads (the storage device itself).  Beside it, the
    same 32 layers' batch kernels with the records in HBM (the kernels' own
    HBM rate)."""
    import tempfile
    import torch
    import oi2
    from oi2.batch_stack import BatchDecodeStack, BatchLayer
    from oi2.filestore import FileStore
    from oi2.synth import zipf_layers
    g = torch.Generator(device=dev).manual_seed(seed)
    t0 = time.time()
    layers = zipf_layers(g, N_LAYERS, INTER, device=dev)
    tmp = tempfile.TemporaryDirectory(dir=ROOT)
    cold_bin = os.path.join(tmp.name, "cold_weights.bin")
    cold_idx = os.path.join(tmp.name, "cold_index.npy")
    w = oi2.format.ColdFileWriter(cold_bin, N_LAYERS)
    for li, l in enumerate(layers):
        w.add_section(li, l.records.cpu().numpy())
    w.close(cold_idx)
    file_gb = os.path.getsize(cold_bin) / 1e9
    log(f"batch 8: {N_LAYERS} Zipf layers and a {file_gb:.2f} GB split file in {time.time() - t0:.1f}s")
    x0 = torch.randn((8, H), generator=g, device=dev).half()
    out = {"tokens_per_step": 8, "layers": N_LAYERS, "n_hot": layers[0].hot.n_hot,
           "file_gb": file_gb, "popularity": "Zipf(1.1) over the intermediate dimension"}
    link = pcie_link_gbs(dev)
    out["h2d_link_gbs_pinned_memcpy"] = link
    for mode, direct in (("page_cache", False), ("direct_io", True)):
        try:
            store = FileStore(cold_bin, cold_idx, direct=direct, threads=READER_THREADS)
        except oi2.OI2Error as e:
            out[mode] = {"error": str(e)}
            continue
        st = BatchDecodeStack([BatchLayer(l.hot, l.lut, l.norm_w, l.predictor, i)
                               for i, l in enumerate(layers)], store, INTER, EPS, "silu", False, 0.0)
        x = x0
        for _ in range(warmup):
            x = st.decode(x)
        torch.cuda.synchronize()
        b0 = st.bytes_read
        t1 = time.perf_counter()
        for _ in range(steps):
            x = st.decode(x)
        torch.cuda.synchronize()
        secs = time.perf_counter() - t1
        rec_bytes = st.bytes_read - b0
        assert torch.isfinite(x.float()).all()
        bound_tok_s = 8 * link * 1e9 / (rec_bytes / steps)
        serial = None
        if not direct:
            serial = host_path_bound(store, layers, rec_bytes / steps / 6400 / N_LAYERS, dev)
        out[mode] = {"tok_s": 8 * steps / secs, "ms_per_step": secs * 1e3 / steps, "steps": steps,
                     "record_bytes_per_step": rec_bytes / steps,
                     "mean_active_cold": rec_bytes / steps / 6400 / N_LAYERS,
                     "file_read_and_h2d_gbs": rec_bytes / secs / 1e9,
                     "reader_threads": READER_THREADS,
                     "pcie_bound_tok_s": bound_tok_s,
                     "frac_of_pcie_bound": 8 * steps / secs / bound_tok_s}
        if serial is not None:
            out[mode]["host_path"] = serial
            out[mode]["frac_of_host_path_bound"] = out[mode]["tok_s"] / serial["bound_tok_s"]
        log(f"batch 8 ({mode}): {out[mode]['tok_s']:.1f} tok/s, {out[mode]['ms_per_step']:.2f} ms/step, "
            f"{out[mode]['mean_active_cold']:.0f} active cold per layer, "
            f"{out[mode]['file_read_and_h2d_gbs']:.2f} GB/s of records from the file, "
            f"{out[mode]['frac_of_pcie_bound']:.3f} of the {bound_tok_s:.0f} tok/s PCIe bound ({link:.1f} GB/s)"
            + (f"; host path: read {serial['read_us_per_layer']:.0f}, copy {serial['h2d_copy_us_per_layer']:.0f}, "
               f"staged {serial['staged_us_per_layer']:.0f} us/layer, {out[mode]['frac_of_host_path_bound']:.3f} "
               f"of its {serial['bound_tok_s']:.0f} tok/s" if serial is not None else ""))
        st.close()
        store.close()
    frac = out["page_cache"]["mean_active_cold"] / (INTER - layers[0].hot.n_hot) \
        if "tok_s" in out.get("page_cache", {}) else 0.15
    k = measure_multi_token(layers, dev, 8, frac, reps=5)
    out["kernels_records_in_hbm"] = k
    log(f"batch 8 kernels alone (records in HBM): {k['us_per_32_layers']:.0f} us per step, "
        f"{k['weight_gbs']:.0f} GB/s ({k['weight_gbs'] / HBM_PEAK_GBS:.3f} of HBM peak)")
    del layers
    tmp.cleanup()
    return out


def _graph_us(fn, dev, reps):
    """Mean microseconds of one replay of a graph capturing fn() (GPU time,
    events on the replay stream), after an eager warm-up call."""
    import torch
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        out = fn()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / reps
    del graph
    return us, out


def measure_config1(dev, reps=20, seed=11, n_layers=32):
    """Config 1: one SwiGLU layer, 2867 hot fp8 neurons with per-row fp32
    scales, the other 11469 cold INT4 records, a fixed uniform-random 10 %
    (1147) of them active, one fp16 token.  The per-layer call
    (oi2_ffn_forward: RMSNorm, hot and cold gate/up, activation, down,
    residual; engine.py:292-312) on n_layers distinct seeded layers chained
    back to back (1.4 GB of weights: no layer's bytes come from a cache),
    captured in one graph; and the same layers through the persistent token
    kernel (a stack of layers without predictors whose records are the
    active ones).  Reported per layer-token."""
    import torch
    from oi2.layer import ColdNeurons, _ffn
    from oi2.stack import DecodeStack, StackLayer
    from oi2.store import ColdSection
    from oi2.synth import SyntheticLayer
    n_hot, n_act = 2867, 1147
    g = torch.Generator(device=dev).manual_seed(seed)
    layers, colds, stack_layers = [], [], []
    for _ in range(n_layers):
        lay = SyntheticLayer(g, INTER, n_hot, std=0.02, device=dev, per_row_scale=True)
        n_cold = lay.records.shape[0]
        slots = torch.randperm(n_cold, generator=g, device=dev)[:n_act].sort().values.int()
        sec = ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut, lay.lut.cpu().numpy(), INTER)
        colds.append(ColdNeurons.from_slots(sec, slots))
        # the stack's layer holds only the active records (ascending id), so
        # its fixed list (every record of the layer) is the same active set
        act_ids = lay.cold_ids[slots.long()]
        lut = torch.full((INTER,), -1, dtype=torch.int32, device=dev)
        lut[act_ids] = torch.arange(n_act, dtype=torch.int32, device=dev)
        stack_layers.append(StackLayer(lay.hot, lay.records[slots.long()].contiguous(), lut, lay.norm_w, None))
        layers.append(lay)
    x0 = torch.randn((1, H), generator=g, device=dev).half()

    def chain():
        x = x0
        for l, c in zip(layers, colds):
            x = _ffn(x, l.norm_w, EPS, l.hot, c, "silu", False, add_residual=True)
        return x

    us, y_call = _graph_us(chain, dev, reps)
    st = DecodeStack(stack_layers, INTER, EPS, "silu", False, 0.0)
    tok_us = None
    y_tok = torch.empty_like(x0[0])
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        st.decode(x0[0], y_tok, stream)
    stream.synchronize()
    st.status(stream)
    same = None
    if st.token_kernel:
        xo = torch.empty_like(x0[0])
        with torch.cuda.stream(stream):
            tok_us = st.profile_token(x0[0], xo, stream, reps=8)
        st.status(stream)
        torch.cuda.synchronize()
        same = bool(torch.equal(xo, y_tok))
    # the two paths agree to the FFN bar (their sums run in other orders)
    a, b = y_call[0].double(), y_tok.double()
    rel = float((a - b).abs().max() / b.abs().max())
    st.close()
    layer_bytes = (n_hot * 3 * H + 2 * n_hot * 4 + H * 4 + n_act * 6400 + 3 * H * 2)
    per = us / n_layers
    out = {"workload": "config 1: one SwiGLU layer 4096x14336, 2867 hot fp8 (per-row scales), "
                       "1147 of 11469 cold INT4 records active (uniform random 10 %), batch 1",
           "layers_timed": n_layers, "bytes_per_layer_token": layer_bytes,
           "per_layer_call": {"us_per_layer_token": per,
                              "hbm_gbs": layer_bytes / (per * 1e-6) / 1e9,
                              "frac_of_hbm_peak": layer_bytes / (per * 1e-6) / 1e9 / HBM_PEAK_GBS,
                              "kernels": "k_ffn_up + k_ffn_down (oi2_ffn_forward), graph-replayed"},
           "ideal_us_at_hbm_peak": layer_bytes / (HBM_PEAK_GBS * 1e9) * 1e6,
           "target_us_at_60pct": layer_bytes / (0.6 * HBM_PEAK_GBS * 1e9) * 1e6,
           "token_kernel_vs_per_layer_call_rel_err": rel}
    if tok_us is not None:
        pt = tok_us / n_layers
        out["token_kernel"] = {"us_per_layer_token": pt, "hbm_gbs": layer_bytes / (pt * 1e-6) / 1e9,
                               "frac_of_hbm_peak": layer_bytes / (pt * 1e-6) / 1e9 / HBM_PEAK_GBS,
                               "kernel": "k_token, the 32 layers in one launch (profile_token)",
                               "profiled_output_equals_decode": same}
    del layers, colds, stack_layers
    return out


def measure_config2(dev, B=64, reps=10, seed=12, n_layers=16):
    """Config 2: one dReLU (TurboSparse-style) layer at 4096x14336,
    y = down(relu(gate x + b) * relu(up x)), gate pre-activations shifted by
    b = -1.3 sigma (sigma = 0.02 sqrt(4096)), 25 % hot fp8, the rest cold
    INT4; a batch of B independent fp16 tokens x ~ N(0, 1) sharing one cold
    set, the union of the tokens' true firing sets (relu(g) relu(u) != 0 over
    the served INT4 weights, profiler.py:130's definition).  n_layers
    distinct seeded layers, each called on the same batch (1.8 GB of weights
    in all), captured in one graph.  Reported per layer call."""
    import math
    import torch
    from oi2 import _lib
    from oi2.layer import ColdNeurons, _ffn, rmsnorm
    from oi2.store import ColdSection
    from oi2.synth import SyntheticLayer
    n_hot = 3584
    sigma = 0.02 * math.sqrt(H)
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((B, H), generator=g, device=dev).half()
    layers, colds, fire_tok, union_n = [], [], [], []
    L = _lib.lib()
    for _ in range(n_layers):
        lay = SyntheticLayer(g, INTER, n_hot, std=0.02, device=dev, gate_bias_shift=-1.3 * sigma)
        n = lay.records.shape[0]
        gate = torch.empty((n, H), dtype=torch.float32, device=dev)
        up = torch.empty((n, H), dtype=torch.float32, device=dev)
        down = torch.empty((H, n), dtype=torch.float32, device=dev)
        allslots = torch.arange(n, dtype=torch.int32, device=dev)
        _lib.check(L.oi2_dequant_records(lay.records.data_ptr(), n, allslots.data_ptr(), n, gate.data_ptr(),
                                         up.data_ptr(), down.data_ptr(), _lib.stream_handle(dev)))
        xn = rmsnorm(x, lay.norm_w, EPS).float()
        fire = (torch.relu(xn @ gate.t() + lay.cold_gate_bias) * torch.relu(xn @ up.t())) != 0
        fire_tok.append(float(fire.float().sum(1).mean()) / n)
        union = fire.any(0).nonzero().flatten().int()
        union_n.append(int(union.numel()))
        del gate, up, down, fire
        sec = ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut, lay.lut.cpu().numpy(), INTER)
        colds.append(ColdNeurons.from_slots(sec, union, gate_bias=lay.cold_gate_bias))
        layers.append(lay)
    torch.cuda.empty_cache()

    def calls():
        return [_ffn(x, l.norm_w, EPS, l.hot, c, "relu", True, add_residual=True)
                for l, c in zip(layers, colds)]

    us, outs = _graph_us(calls, dev, reps)
    assert all(torch.isfinite(o.float()).all() for o in outs)
    per = us / n_layers
    mean_union = sum(union_n) / n_layers
    layer_bytes = (n_hot * 3 * H + 3 * n_hot * 4 + H * 4 + mean_union * (6400 + 4) + 2 * B * H * 2 + H * 2)
    flop = 2 * B * H * (n_hot + mean_union) * 3
    out = {"workload": f"config 2: one dReLU layer 4096x14336, gate bias -1.3 sigma, 3584 hot fp8, "
                       f"batch {B} of independent tokens over the union of their true firing sets",
           "layers_timed": n_layers, "batch": B,
           "firing_per_token_frac_of_cold": sum(fire_tok) / n_layers,
           "union_records_mean": mean_union,
           "union_frac_of_cold": mean_union / (INTER - n_hot),
           "us_per_layer": per, "bytes_per_layer": layer_bytes,
           "hbm_gbs": layer_bytes / (per * 1e-6) / 1e9,
           "frac_of_hbm_peak": layer_bytes / (per * 1e-6) / 1e9 / HBM_PEAK_GBS,
           "ideal_us_at_hbm_peak": layer_bytes / (HBM_PEAK_GBS * 1e9) * 1e6,
           "tflops": flop / (per * 1e-6) / 1e12,
           "frac_of_fp16_dense_peak": flop / (per * 1e-6) / 1e12 / 2500.0,
           "kernels": "oi2_ffn_forward at batch 64 (matrix-core batch kernels), graph-replayed"}
    del layers, colds
    return out


def host_path_bound(store, layers, n_act, dev, reps=3):
    """The host side of config 4 alone, per layer: the file store's read of
    n_act ascending records (page cache -> pinned buffer), one pinned ->
    device copy of those bytes, and the staged call the decode makes (the
    read in chunks with each finished run's copy enqueued behind it, waited
    for at the end of every layer).  The read and the device copy share the
    host's memory bandwidth, so the staged call, not the larger of the two,
    bounds the step."""
    import numpy as np
    import torch
    n = int(round(n_act))
    rng = np.random.default_rng(0)
    host = torch.empty(n * 6400, dtype=torch.uint8).pin_memory()
    dst = torch.empty(n * 6400, dtype=torch.uint8, device=dev)
    n_rec = int(layers[0].records.shape[0])
    sets = [np.sort(rng.choice(n_rec, n, replace=False)).astype(np.int32) for _ in range(N_LAYERS)]
    stream = torch.cuda.Stream(device=dev)
    best_r = best_c = best_s = float("inf")
    for _ in range(reps):
        t0 = time.perf_counter()
        for L in range(N_LAYERS):
            store.read(L, sets[L], host)
        best_r = min(best_r, (time.perf_counter() - t0) / N_LAYERS)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for L in range(N_LAYERS):
            dst.copy_(host, non_blocking=True)
        torch.cuda.synchronize()
        best_c = min(best_c, (time.perf_counter() - t0) / N_LAYERS)
        t0 = time.perf_counter()
        for L in range(N_LAYERS):
            store.stage(L, sets[L], host, dst, stream)
            stream.synchronize()
        best_s = min(best_s, (time.perf_counter() - t0) / N_LAYERS)
    return {"records_per_layer": n, "read_us_per_layer": best_r * 1e6, "read_gbs": n * 6400 / best_r / 1e9,
            "h2d_copy_us_per_layer": best_c * 1e6, "h2d_copy_gbs": n * 6400 / best_c / 1e9,
            "staged_us_per_layer": best_s * 1e6, "staged_gbs": n * 6400 / best_s / 1e9,
            "bound_tok_s": 8 / (N_LAYERS * best_s)}


def measure_multi_token(layers, dev, M, frac, reps, seed=1):
    """M tokens through the 32 layers on the matrix-core path (batch decode at
    small M, a prefill chunk at M = 512): each layer's cold half is a fixed
    random `frac` of its cold neurons (the batch's union).  The 32-layer
    chain is captured once in a graph and replayed, so `us` is GPU time."""
    import torch
    from oi2.layer import ColdNeurons, _ffn
    from oi2.store import ColdSection
    g = torch.Generator(device=dev).manual_seed(seed)
    colds = []
    for l in layers:
        n = l.records.shape[0]
        slots = torch.randperm(n, generator=g, device=dev)[: int(frac * n)].int()
        sec = ColdSection(0, l.cold_ids.cpu().numpy(), l.records, l.lut, l.lut.cpu().numpy(), INTER)
        colds.append(ColdNeurons.from_slots(sec, slots))
    x0 = torch.randn((M, H), generator=g, device=dev).half()
    stream = torch.cuda.Stream(device=dev)

    def separate(x):
        for l, c in zip(layers, colds):
            x = _ffn(x, l.norm_w, EPS, l.hot, c, "silu", False, add_residual=True)
        return x

    def chained(x):
        # from 17 tokens each call's final add writes the next layer's
        # normalised rows (oi2_ffn_forward_chain): one launch fewer per layer
        xn = None
        for i, (l, c) in enumerate(zip(layers, colds)):
            nxt = layers[i + 1].norm_w if i + 1 < len(layers) else None
            r = _ffn(x, l.norm_w, EPS, l.hot, c, "silu", False, add_residual=True, xn_in=xn, next_norm_w=nxt)
            x, xn = r if nxt is not None else (r, None)
        return x

    def timed(chain):
        with torch.cuda.stream(stream):
            chain(x0)                                   # warm (workspaces, library)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = chain(x0)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us_ = e0.elapsed_time(e1) * 1e3 / reps
        del graph
        return us_, y

    us_sep, y_sep = timed(separate)
    us, y = timed(chained) if M > 16 else (us_sep, y_sep)
    assert torch.equal(y, y_sep), "the chained calls must give the separate calls' bits"
    n_hot = layers[0].hot.n_hot
    n_act = int(frac * (INTER - n_hot))
    flop = N_LAYERS * 2 * M * H * (n_hot + n_act) * 3
    weight_bytes = N_LAYERS * (3 * n_hot * H + n_act * 6400)
    assert torch.isfinite(y.float()).all()
    return {"tokens": M, "active_cold_frac": frac, "us_per_32_layers": us,
            "separate_calls_us_per_32_layers": us_sep,
            "tok_s": M / (us * 1e-6), "tflops": flop / (us * 1e-6) / 1e12,
            "mfma_frac_fp16_dense": flop / (us * 1e-6) / 2.5e15,
            "weight_gbs": weight_bytes / (us * 1e-6) / 1e9}


def attention_layers(dev, g, n_kv=8):
    """32 GroupedQueryAttention layers of Mistral-7B geometry from seeded
    N(0, 0.02) weights cast to fp8 e4m3fn, as splitter.py:175-177 stores them."""
    import torch
    import oi2
    cfg = {"num_attention_heads": 32, "num_key_value_heads": n_kv, "hidden_dim": H,
           "rms_norm_eps": EPS}
    layers = []
    for li in range(N_LAYERS):
        p = f"layer_{li:03d}."

        def w(r, c):
            return (torch.randn((r, c), generator=g, device=dev) * 0.02).to(torch.float8_e4m3fn)
        wd = {p + "q_proj": w(H, H), p + "k_proj": w(n_kv * 128, H), p + "v_proj": w(n_kv * 128, H),
              p + "o_proj": w(H, H),
              p + "input_layernorm": (1.0 + 0.05 * torch.randn(H, generator=g, device=dev)).half()}
        layers.append(oi2.GroupedQueryAttention(li, wd, cfg))
    return layers


def measure_decode_step(ffn_layers_syn, thr, dev, ctx=512, reps=20, seed=7):
    """A whole decode step of the 32 layers, attention and FFN, in
    DesdemonaEngine.forward's order (engine.py:421-438) through oi2.DecoderStep:
    batch 1, each layer's KV cache holding `ctx` positions, the cold records
    in HBM, each layer's cold set predicted from the previous layer's
    post-attention state.  Two FFN sides over the same synthetic layers: the
    drop-in SparseFFNLayers (predictor, then FFN, per layer) and a DecodeStack
    (one layer per oi2_stack_layer call: FFN and the next layer's prediction
    in two kernels).  Each step is captured in one graph and replayed."""
    import math
    import torch
    import oi2
    from oi2.decode_step import DecoderStep
    from oi2.stack import DecodeStack, StackLayer
    from oi2.store import ColdSection
    g = torch.Generator(device=dev).manual_seed(seed)
    attn = attention_layers(dev, g)

    class _Sections:                  # the store interface SparseFFNLayer reads
        residency = "hbm"

        def __init__(self, lay):
            self.sec = ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut,
                                   lay.lut.cpu().numpy(), INTER)

        def section(self, layer_idx, expert_idx=0):
            return self.sec

    cfg = {"hidden_act": "silu", "intermediate_dim": INTER, "rms_norm_eps": EPS, "hidden_dim": H}
    p_thr = 1.0 / (1.0 + math.exp(-thr))
    ffn = [oi2.SparseFFNLayer(li, "", _Sections(l), l.predictor, cfg, dev, hot=l.hot,
                              ffn_norm_weight=l.norm_w, threshold=p_thr)
           for li, l in enumerate(ffn_layers_syn)]
    stack = DecodeStack([StackLayer(l.hot, l.records, l.lut, l.norm_w, l.predictor) for l in ffn_layers_syn],
                        INTER, EPS, "silu", False, thr)
    stack.set_expected_active(int(1.3 * ACTIVE_FRAC * (INTER - N_HOT)))
    cos, sin = oi2.rope_tables(ctx + 1, 128, 1e6, device=dev)
    c1, s1 = cos[ctx:ctx + 1], sin[ctx:ctx + 1]
    x0 = torch.randn((1, 1, H), generator=g, device=dev).half()
    caches = []
    for _ in attn:
        k = torch.randn((1, 8, ctx, 128), generator=g, device=dev).half()
        caches.append((k, torch.randn_like(k)))
    out = {"layers": N_LAYERS, "batch": 1, "context": ctx}
    for name, ffn_side in (("drop_in_layers", ffn), ("stack_layers", stack)):
        step = DecoderStep(attn, ffn_side)
        stream = torch.cuda.Stream(device=dev)
        with torch.cuda.stream(stream):
            _, kv = step(x0, c1, s1, caches)          # copies the caches into the layers' buffers
            kvs = [(k[:, :, :ctx], v[:, :, :ctx]) for k, v in kv]
            for a in attn:                            # decode position ctx again, in place
                a.rewind(ctx)
            step(x0, c1, s1, kvs)
        stream.synchronize()
        for a in attn:
            a.rewind(ctx)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y, _ = step(x0, c1, s1, kvs)
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        assert torch.isfinite(y.float()).all()
        del graph
        out[name] = {"us_per_token": us, "us_per_layer": us / N_LAYERS, "tok_s": 1e6 / us}
    stack.close()
    out["path"] = ("DecoderStep: GroupedQueryAttention (3 kernels per layer) + FFN per layer as the "
                   "drop-in SparseFFNLayer (predictor 3 kernels, FFN 3) or DecodeStack.layer "
                   "(3 kernels with the next layer's prediction fused); one graph per token")
    return out


def measure_attention(dev, contexts=(512, 4096), reps=20, seed=6):
    """Decode attention (engine.py:63-125) at batch 1 through 32 layers of Mistral-7B geometry (32 query / 8 kv
    heads of 128, fp8 projections): each layer's cache holds `ctx` positions
    and the token attends to ctx + 1.  The 32 calls are captured in one graph
    and replayed, so the time is GPU time.  Algorithmic bytes per layer: the
    fp8 q/k/v/o weights (41.9 MB) plus the K and V rows read (4096 B per
    position) plus the new rows and the token."""
    import torch
    import oi2
    n_kv = 8
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = attention_layers(dev, g, n_kv)
    out = {"layers": N_LAYERS, "batch": 1, "n_q": 32, "n_kv": n_kv, "head_dim": 128,
           "weight_bytes_per_layer": (H + 2 * n_kv * 128) * H + H * H}
    stream = torch.cuda.Stream(device=dev)
    for ctx in contexts:
        cos, sin = oi2.rope_tables(ctx + 1, 128, 1e6, device=dev)
        caches = []
        for a in layers:
            k = torch.randn((1, n_kv, ctx, 128), generator=g, device=dev).half()
            caches.append((k, torch.randn_like(k)))
        x0 = torch.randn((1, 1, H), generator=g, device=dev).half()
        res = [torch.empty_like(x0) for _ in range(2)]
        c1, s1 = cos[ctx:ctx + 1], sin[ctx:ctx + 1]
        # the first call copies each cache into its layer's buffer; later
        # calls pass back the views (in-place append at position ctx)
        kvs = []
        with torch.cuda.stream(stream):
            for a, kv in zip(layers, caches):
                _, kv2 = a(x0, c1, s1, kv)
                kvs.append((kv2[0][:, :, :ctx], kv2[1][:, :, :ctx]))
        stream.synchronize()

        def chain():
            x = x0
            for i, (a, kv) in enumerate(zip(layers, kvs)):
                a(x, c1, s1, kv, residual_out=res[i & 1])
                x = res[i & 1]
            return x
        # every replay decodes position ctx again, in place: each layer's
        # cache is rolled back to ctx positions before the calls
        for a in layers:
            a.rewind(ctx)
        with torch.cuda.stream(stream):
            chain()
        stream.synchronize()
        for a in layers:
            a.rewind(ctx)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = chain()
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / reps
        assert torch.isfinite(y.float()).all()
        per_layer = out["weight_bytes_per_layer"] + (ctx + 1) * 2 * n_kv * 128 * 2 + 3 * H * 2
        gbs = N_LAYERS * per_layer / (us * 1e-6) / 1e9
        out[f"ctx{ctx}"] = {"us_per_32_layers": us, "us_per_layer": us / N_LAYERS,
                            "bytes_per_layer": per_layer, "gbs": gbs, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS,
                            "tok_s_attention_only": 1e6 / us}
        log(f"attention ctx {ctx}: {us / N_LAYERS:.2f} us/layer, {gbs:.0f} GB/s ({gbs / HBM_PEAK_GBS:.3f} of HBM)")
        del graph, caches, kvs
    del layers
    return out


def measure_gemm_reference(dev, n=8192, reps=10):
    """The attainable fp16 matrix rate on this GPU: a vendor-library
    (hipBLASLt through torch.matmul) n x n x n fp16 GEMM, fp32 accumulate."""
    import torch
    a = torch.randn((n, n), device=dev).half()
    b = torch.randn((n, n), device=dev).half()
    for _ in range(2):
        torch.matmul(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.matmul(a, b)
    e1.record()
    torch.cuda.synchronize()
    s = e0.elapsed_time(e1) / 1e3 / reps
    return 2.0 * n ** 3 / s / 1e12


def measure_split_writer(dev, reps=5):
    """The device split writer on one full layer: 10752 cold neurons of a
    (14336, 4096) gate/up and (4096, 14336) down in fp32, quantised and framed
    as one cold_weights.bin section; plus the restated reference quantiser
    (one vector at a time, as splitter.py:229-247 does) on a CPU sample."""
    import numpy as np
    import torch
    from oi2.split import quantize_section
    from oracle import oracle as O
    g = torch.Generator(device=dev).manual_seed(5)
    gate = torch.randn((INTER, H), generator=g, device=dev) * 0.02
    up = torch.randn((INTER, H), generator=g, device=dev) * 0.02
    down = torch.randn((H, INTER), generator=g, device=dev) * 0.02
    cold = np.arange(N_HOT, INTER)
    sec = quantize_section(0, gate, up, down, cold)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        sec = quantize_section(0, gate, up, down, cold)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    n = cold.size
    in_bytes = n * 3 * H * 4
    # CPU: the reference quantises each neuron's three vectors in turn
    sample = 48
    vecs = [(gate[i].cpu().numpy(), up[i].cpu().numpy(), down[:, i].cpu().numpy())
            for i in range(N_HOT, N_HOT + sample)]
    t0 = time.perf_counter()
    for gv, uv, dv in vecs:
        for v in (gv, uv, dv):
            O.quantize_int4_ref(v)
    cpu_s = (time.perf_counter() - t0) / sample
    del gate, up, down, sec
    return {"neurons": int(n), "ms_per_layer": ms, "neurons_per_s": n / (ms * 1e-3),
            "input_gbs": in_bytes / (ms * 1e-3) / 1e9,
            "section_bytes": int(16 + n * 6400),
            "model_32_layers_s": N_LAYERS * ms / 1e3,
            "cpu_port_us_per_neuron": cpu_s * 1e6,
            "cpu_port_model_32_layers_s": cpu_s * n * N_LAYERS,
            "cpu_sample": f"{sample} neurons x 3 vectors through the restated quantize_int4, 1 thread"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--profile-reps", type=int, default=8)
    ap.add_argument("--cpu-tokens", type=int, default=6)
    ap.add_argument("--no-multi-token", dest="multi_token", action="store_false",
                    help="skip the 8 / 64 / 512-token matrix-core measurements")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-split-writer", dest="split_writer", action="store_false",
                    help="skip the device split writer measurement")
    ap.add_argument("--no-cold-dequant", dest="cold_dequant", action="store_false",
                    help="skip the cold INT4 dequant GB/s measurement")
    ap.add_argument("--no-batch8", dest="batch8", action="store_false",
                    help="skip the batch-8 Zipf decode with the records read from the file")
    ap.add_argument("--batch8-steps", type=int, default=8)
    ap.add_argument("--no-attention", dest="attention", action="store_false",
                    help="skip the decode-attention leg")
    ap.add_argument("--attention-only", action="store_true")
    ap.add_argument("--multi-token-only", action="store_true",
                    help="only the multi-token (batch decode / prefill) leg")
    ap.add_argument("--batch8-only", action="store_true",
                    help="only the batch-8 Zipf decode with the records read from the file (config 4)")
    ap.add_argument("--configs-only", action="store_true",
                    help="only the single-layer legs: config 1 (bs1 SwiGLU) and config 2 (B=64 dReLU)")
    ap.add_argument("--no-configs", dest="configs", action="store_false",
                    help="skip the single-layer config 1 / config 2 legs")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MiB device copy 8 times (the reference kernel "
                         "for scaling FETCH_SIZE / WRITE_SIZE counter readings) and exit")
    ap.add_argument("--hbm-only", action="store_true",
                    help="only the HBM-resident token kernel leg (for profiling k_token)")
    ap.add_argument("--cold-only", action="store_true",
                    help="only the cold INT4 dequant measurement (for profiling the cold kernels)")
    ap.add_argument("--token-phases", type=int, default=0, metavar="TOKENS",
                    help="only trace the persistent token kernel's phases over TOKENS tokens "
                         "(per-group s_memrealtime stamps) and print their summary")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    import oi2  # noqa: F401
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(8):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copied {src.numel() * 4} bytes 8 times")
        return
    if args.attention_only:
        res = measure_attention(dev)
        layers, st, thr, g = build_stack(args.seed, dev)
        res["full_decode_step"] = measure_decode_step(layers, thr, dev)
        for side in ("drop_in_layers", "stack_layers"):
            log(f"full decode step ({side}): {res['full_decode_step'][side]['us_per_token']:.0f} us/token")
        print(json.dumps({"attention": res}), flush=True)
        return
    if args.batch8_only:
        print(json.dumps({"batch8_file": measure_batch8_file(dev, args.batch8_steps, 2)}), flush=True)
        return
    if args.configs_only:
        c1 = measure_config1(dev)
        log(f"config 1: {c1['per_layer_call']['us_per_layer_token']:.2f} us per layer-token per call "
            f"({c1['per_layer_call']['frac_of_hbm_peak']:.3f} of HBM)"
            + (f", token kernel {c1['token_kernel']['us_per_layer_token']:.2f} us "
               f"({c1['token_kernel']['frac_of_hbm_peak']:.3f})" if "token_kernel" in c1 else ""))
        c2 = measure_config2(dev)
        log(f"config 2: {c2['us_per_layer']:.1f} us per layer, union {c2['union_frac_of_cold']:.3f} of cold, "
            f"{c2['frac_of_hbm_peak']:.3f} of HBM")
        print(json.dumps({"config1": c1, "config2": c2}), flush=True)
        return
    t0 = time.time()
    layers, st, thr, g = build_stack(args.seed, dev)
    torch.cuda.synchronize()
    log(f"built 32-layer stack in {time.time() - t0:.1f}s, threshold logit {thr:.4f}")
    if args.cold_only:
        cold = measure_cold_dequant(layers, dev)
        print(json.dumps({"cold_dequant": cold}), flush=True)
        return
    if args.token_phases:
        print(json.dumps({"token_phases": measure_token_phases(st, g, dev, args.token_phases)}), flush=True)
        return
    if args.multi_token_only:
        multi = {}
        for M, frac in ((8, 0.15), (64, 0.50), (512, 0.40), (1024, 0.40)):
            multi[f"m{M}"] = measure_multi_token(layers, dev, M, frac, reps=5)
            log(f"{M} tokens x 32 layers: {multi[f'm{M}']['us_per_32_layers']:.0f} us "
                f"(separate calls {multi[f'm{M}']['separate_calls_us_per_32_layers']:.0f} us)")
        print(json.dumps({"multi_token": multi}), flush=True)
        return
    stream = torch.cuda.Stream(device=dev)
    x0 = torch.randn(H, generator=g, device=dev).half()

    # ---- the headline: config 3, cold store in pinned host memory, staged ----
    staged = None
    if not args.hbm_only:
        sst, pinned = build_staged(layers, thr)
        secs, x_last = timed_decode(sst, x0, stream, args.warmup, args.steps)
        tok_s = args.steps / secs
        log(f"staged: timed {args.steps} tokens in {secs * 1e3:.2f} ms ({tok_s:.1f} tok/s)")
        # the bytes each token moves: the active records of the timed tokens
        # themselves, replayed from the same start (each token's sets follow
        # from its input alone, and the decode is deterministic)
        active_st, x_replay = mean_active_over(sst, advance(sst, x0, stream, args.warmup), stream, args.steps)
        replay_same = bool(torch.equal(x_replay, x_last))
        with torch.cuda.stream(stream):
            copy_us = sst.profile_staging(x0, torch.empty_like(x0), stream, reps=2)
        torch.cuda.synchronize()
        link = pcie_link_gbs(dev)
        h2d_bytes = N_LAYERS * active_st * 6400
        staged = {"tok_s": tok_s, "ms_per_token": secs * 1e3 / args.steps, "steps": args.steps,
                  "store": "pinned host memory (hipHostMalloc via torch pin_memory), 32 x 68.8 MB",
                  "copy_workgroups": COPY_WORKGROUPS,
                  "copy_alone_us_per_layer": copy_us,
                  "copy_alone_gbs": active_st * 6400 / (copy_us * 1e-6) / 1e9,
                  "h2d_bytes_per_token": h2d_bytes,
                  "h2d_gbs_end_to_end": h2d_bytes * tok_s / 1e9,
                  "h2d_link_gbs_pinned_memcpy": link,
                  "pcie_bound_tok_s": link * 1e9 / h2d_bytes,
                  "frac_of_pcie_bound": tok_s / (link * 1e9 / h2d_bytes),
                  "mean_active_cold": active_st,
                  "active_counted_on": f"the {args.steps} timed tokens, replayed (same output bits: {replay_same})"}
        log(f"staged: {tok_s:.1f} tok/s = {staged['frac_of_pcie_bound']:.3f} of the PCIe bound "
            f"({staged['pcie_bound_tok_s']:.1f} tok/s at {link:.1f} GB/s); copy alone {copy_us:.1f} us/layer")
        sst.close()
        del pinned

    # ---- the same workload with the records in HBM: the token kernel ----
    secs_h, xi = timed_decode(st, x0, stream, args.warmup, args.steps)
    hbm_tok_s = args.steps / secs_h
    log(f"HBM-resident: timed {args.steps} tokens in {secs_h * 1e3:.2f} ms ({hbm_tok_s:.1f} tok/s)")
    token_path = st.token_kernel
    two_tok_s = None
    if token_path:
        st.set_token_kernel(False)
        s2, _ = timed_decode(st, x0, stream, 4, min(args.steps, 128))
        two_tok_s = min(args.steps, 128) / s2
        st.set_token_kernel(True)
        log(f"two-launch path: {two_tok_s:.1f} tok/s")
    xo = torch.empty_like(xi)
    tok_us = None
    with torch.cuda.stream(stream):
        if token_path:
            tok_us = st.profile_token(xi, xo, stream, reps=args.profile_reps)
        up_us, down_us = st.profile(xi, xo, stream, reps=args.profile_reps)
    st.status(stream)
    xs, counts, slots, ids = st.trace()
    torch.cuda.synchronize()
    c = counts.sum(1).cpu().tolist()
    up_b = sum(up_launch_bytes(c[L]) for L in range(N_LAYERS)) / N_LAYERS
    down_b = sum(down_launch_bytes(c[L + 1] if L + 1 < N_LAYERS else 0)
                 for L in range(N_LAYERS)) / N_LAYERS
    up_gbs = up_b / (up_us * 1e-6) / 1e9
    down_gbs = down_b / (down_us * 1e-6) / 1e9
    mean_active = sum(c) / N_LAYERS
    token_bytes = N_LAYERS * (up_b + down_b)
    log(f"ffn_up {up_us:.2f} us/launch {up_gbs:.0f} GB/s; ffn_down {down_us:.2f} us "
        f"{down_gbs:.0f} GB/s; mean active cold {mean_active:.0f}")
    if token_path:
        tok_gbs = token_bytes / (tok_us * 1e-6) / 1e9
        log(f"token kernel {tok_us:.1f} us/launch {tok_gbs:.0f} GB/s ({token_bytes / 1e6:.1f} MB)")
        roofline = {"bound": "hbm", "achieved": tok_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": tok_gbs / HBM_PEAK_GBS, "traffic": TOKEN_TRAFFIC_BYTES,
                    "traffic_source": TOKEN_TRAFFIC_SOURCE, "kernel": "k_token",
                    "us_per_launch": tok_us, "bytes_per_launch": token_bytes,
                    "workload": "the same 32 layers with the cold records in HBM (hbm_resident): "
                                "the decode kernel on its own; the staged headline is bound by PCIe, "
                                "see staging"}
    else:
        roofline = {"bound": "hbm", "achieved": up_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": up_gbs / HBM_PEAK_GBS, "traffic": None, "kernel": "k_ffn_up",
                    "us_per_launch": up_us, "bytes_per_launch": up_b}
    hbm_resident = {"tok_s": hbm_tok_s, "ms_per_token": secs_h * 1e3 / args.steps,
                    "path": "token kernel" if token_path else "two launches per layer",
                    "two_launch_tok_s": two_tok_s, "token_bytes": token_bytes,
                    "hbm_frac_end_to_end": token_bytes * hbm_tok_s / (HBM_PEAK_GBS * 1e9),
                    "cold_neurons_per_s": mean_active * N_LAYERS * hbm_tok_s,
                    "mean_active_cold": mean_active,
                    "kernels": {"k_ffn_up": {"us_per_launch": up_us, "achieved_gbs": up_gbs,
                                             "bytes_per_launch": up_b},
                                "k_ffn_down": {"us_per_launch": down_us, "achieved_gbs": down_gbs,
                                               "bytes_per_launch": down_b}}}

    cold = None
    if args.cold_dequant and not args.hbm_only:
        cold = measure_cold_dequant(layers, dev)
        f, r = cold["fused_cold_ffn"], cold["read_neurons_dequant"]
        log(f"cold INT4 fused gather/dequant/FFN: {f['records']} records in {f['us_per_layer']:.1f} us "
            f"= {f['record_gbs']:.0f} GB/s of records ({f['frac_of_hbm_peak']:.3f} of HBM peak); "
            f"read_neurons dequant {r['records']} records in {r['us']:.1f} us "
            f"({r['hbm_gbs_records_plus_fp32_out']:.0f} GB/s with its fp32 output)")

    multi = None
    if args.multi_token and not args.hbm_only:
        multi = {"fp16_gemm_ref_tflops": measure_gemm_reference(dev)}
        log(f"vendor fp16 GEMM 8192^3: {multi['fp16_gemm_ref_tflops']:.0f} TFLOP/s")
        for M, frac in ((8, 0.15), (64, 0.50), (512, 0.40), (1024, 0.40)):
            r = measure_multi_token(layers, dev, M, frac, reps=5)
            r["frac_of_fp16_gemm_ref"] = r["tflops"] / multi["fp16_gemm_ref_tflops"]
            multi[f"m{M}"] = r
            log(f"{M} tokens x 32 layers: {r['us_per_32_layers']:.0f} us, "
                f"{r['tflops']:.1f} TFLOP/s, {r['weight_gbs']:.0f} GB/s"
                + (f" (chained calls; separate calls {r['separate_calls_us_per_32_layers']:.0f} us)"
                   if M > 16 else ""))

    config1 = config2 = None
    if args.configs and not args.hbm_only:
        config1 = measure_config1(dev)
        log(f"config 1: {config1['per_layer_call']['us_per_layer_token']:.2f} us per layer-token per call "
            f"({config1['per_layer_call']['frac_of_hbm_peak']:.3f} of HBM)"
            + (f", token kernel {config1['token_kernel']['us_per_layer_token']:.2f} us "
               f"({config1['token_kernel']['frac_of_hbm_peak']:.3f})" if "token_kernel" in config1 else ""))
        config2 = measure_config2(dev)
        log(f"config 2: {config2['us_per_layer']:.1f} us per layer, union {config2['union_frac_of_cold']:.3f} "
            f"of cold, {config2['frac_of_hbm_peak']:.3f} of HBM")

    batch8 = None
    if args.batch8 and not args.hbm_only:
        batch8 = measure_batch8_file(dev, args.batch8_steps, 2)

    attention = None
    if args.attention and not args.hbm_only:
        attention = measure_attention(dev)
        attention["full_decode_step"] = measure_decode_step(layers, thr, dev)
        f = attention["full_decode_step"]
        for side in ("drop_in_layers", "stack_layers"):
            log(f"full decode step (attention + FFN as {side}, ctx {f['context']}): "
                f"{f[side]['us_per_token']:.0f} us/token, {f[side]['tok_s']:.0f} tok/s")

    writer = None
    if args.split_writer and not args.hbm_only:
        writer = measure_split_writer(dev)
        log(f"split writer: {writer['neurons']} cold neurons in {writer['ms_per_layer']:.2f} ms "
            f"({writer['input_gbs']:.0f} GB/s of fp32 input); restated CPU quantiser "
            f"{writer['cpu_port_us_per_neuron']:.0f} us/neuron")

    cpu = None
    if not args.no_cpu_baseline and args.cpu_tokens > 0 and not args.hbm_only:
        tokens = []
        x = xi.clone()
        y = torch.empty_like(x)
        for t in range(args.cpu_tokens):
            with torch.cuda.stream(stream):
                st.decode(x, y, stream)
            stream.synchronize()
            xs, counts, slots, ids = st.trace()
            torch.cuda.synchronize()
            xs_in = [x.clone()] + [xs[i].clone() for i in range(N_LAYERS - 1)]
            tokens.append((xs_in, [st.active_ids(L, counts, ids) for L in range(N_LAYERS)]))
            x, y = y.clone(), x
        cpu = cpu_baseline(layers, tokens, args.cpu_seconds)
        log(f"cpu baseline {cpu['value']:.4f} tok/s over {cpu['seconds']:.1f}s, "
            f"{cpu['cold_neurons_per_s']:.0f} cold neurons/s")

    if staged is not None:
        value, secs_v, steps_v = staged["tok_s"], staged["ms_per_token"] * args.steps / 1e3, args.steps
        workload = ("32-layer 4096x14336 SwiGLU hot/cold FFN decode, batch 1, 25% hot fp8 in HBM, "
                    "cold INT4 records in pinned host memory staged into HBM over PCIe one layer "
                    "ahead, bf16 predictor at 5% active")
    else:
        value, secs_v, steps_v = hbm_tok_s, secs_h, args.steps
        workload = ("32-layer 4096x14336 SwiGLU hot/cold FFN decode, batch 1, 25% hot fp8 in HBM, "
                    "cold INT4 records in HBM, bf16 predictor at 5% active")
    out = {
        "metric": "FFN decode tok/s (32L, 4096x14336, bs1); cold INT4 dequant GB/s vs HBM",
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": steps_v,
        "warmup": args.warmup,
        "ms_per_step": secs_v * 1e3 / steps_v,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3+int4 weights, fp16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,0.02) weights, random-init bf16 predictors)",
        "config": {"workload": workload, "layers": N_LAYERS, "hidden": H, "intermediate": INTER,
                   "n_hot": N_HOT, "batch": 1,
                   "mean_active_cold": round(staged["mean_active_cold"] if staged is not None
                                             else mean_active, 1),
                   "parallelism": "single GPU"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "staging": staged,
        "hbm_resident": hbm_resident,
        "cold_dequant": cold,
        "config1": config1,
        "config2": config2,
        "batch8_file": batch8,
        "multi_token": multi,
        "split_writer": writer,
        "attention": attention,
    }
    if cpu is not None and cold is not None:
        out["cold_dequant"]["gpu_vs_cpu_cold_neurons"] = (
            cold["fused_cold_ffn"]["neurons_per_s"] / cpu["cold_neurons_per_s"])
    print(json.dumps(out), flush=True)
    st.close()


if __name__ == "__main__":
    main()
