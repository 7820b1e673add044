"""The reference's CPU cold path, restated for the cpu_baseline leg of
bench.py.

TEST INFRASTRUCTURE ONLY (timed baseline, never shipped).

It keeps the reference's cost structure on purpose: one Python iteration per
requested neuron, three ``bytes`` slices of the mapped file and three
``torch.frombuffer`` scale reads per neuron (splitter.py:369-391), the
per-vector torch dequant (splitter.py:111-124), ``torch.stack`` of the rows
(splitter.py:400-402), then the FFN halves with ``F.linear``
(engine.py:194-205).  The hot half runs in fp32 here (the reference runs it in
fp16, which is slower on a CPU), so the baseline is, if anything, flattering.
"""
from __future__ import annotations

import time

import numpy as np
import torch
import torch.nn.functional as F

VEC = 2048
SCALES = 64


def dequantize_int4(packed: bytes, scales: torch.Tensor, N: int, group: int = 128):
    """splitter.py:111-124: nibbles -> signed int -> float times group scale."""
    b = np.frombuffer(packed, dtype=np.uint8)
    lo = torch.tensor(b & 0x0F, dtype=torch.int8)
    hi = torch.tensor((b >> 4) & 0x0F, dtype=torch.int8)
    v = torch.stack([lo, hi], dim=1).reshape(-1)[:N].float()
    v = torch.where(v > 7, v - 16, v)
    n_groups = (N + group - 1) // group
    return v * scales[:n_groups].repeat_interleave(group)[:N]


def read_neurons(buf, id_to_offset: dict, neuron_ids, H: int = 4096):
    """splitter.py:354-403 over an in-memory buffer (bytes / mmap / memoryview)."""
    g_rows, u_rows, d_rows = [], [], []
    for nid in neuron_ids:
        if nid not in id_to_offset:
            continue
        off = id_to_offset[nid] + 2
        gb = bytes(buf[off: off + VEC])
        ub = bytes(buf[off + VEC: off + 2 * VEC])
        db = bytes(buf[off + 2 * VEC: off + 3 * VEC])
        so = off + 3 * VEC
        gs = torch.frombuffer(bytearray(buf[so: so + SCALES]), dtype=torch.float16).float()
        us = torch.frombuffer(bytearray(buf[so + SCALES: so + 2 * SCALES]), dtype=torch.float16).float()
        ds = torch.frombuffer(bytearray(buf[so + 2 * SCALES: so + 3 * SCALES]),
                              dtype=torch.float16).float()
        g_rows.append(dequantize_int4(gb, gs, H))
        u_rows.append(dequantize_int4(ub, us, H))
        d_rows.append(dequantize_int4(db, ds, H))
    if not g_rows:
        return None
    return torch.stack(g_rows), torch.stack(u_rows), torch.stack(d_rows, dim=1)


def ffn(x, hot, cold, activation="silu", act_on_both=False):
    """engine.py:194-209 on the CPU: hot (gate, up, down) and cold (gate, up,
    down) dense fp32 tensors, down stored (H, n)."""
    act = F.relu if activation == "relu" else F.silu
    out = torch.zeros_like(x)
    for half in (hot, cold):
        if half is None:
            continue
        g, u, d = half
        gg, uu = F.linear(x, g), F.linear(x, u)
        h = act(gg) * (act(uu) if act_on_both else uu)
        out = out + F.linear(h, d)
    return out


def time_layers(samples, threads: int = 1):
    """Time the restated per-layer path over ``samples`` = list of
    (x_n (1,H) fp32, hot dense tuple, buf, id_to_offset, cold ids).  Returns
    (seconds, seconds spent in the cold fetch + dequant, neurons fetched,
    per-call seconds of each layer call, per-call seconds of its cold fetch)."""
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        neurons = 0
        t_cold = 0.0
        calls, fetches = [], []
        t0 = time.perf_counter()
        for xn, hot, buf, offs, ids in samples:
            t1 = time.perf_counter()
            cold = read_neurons(buf, offs, ids)
            t2 = time.perf_counter()
            t_cold += t2 - t1
            neurons += 0 if cold is None else cold[0].shape[0]
            ffn(xn, hot, cold)
            calls.append(time.perf_counter() - t1)
            fetches.append(t2 - t1)
        dt = time.perf_counter() - t0
    finally:
        torch.set_num_threads(prev)
    return dt, t_cold, neurons, calls, fetches
