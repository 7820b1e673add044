"""Seeded synthetic hot/cold models for the benchmark and the tests.

Weights are drawn N(0, std) from a seeded torch generator on the target
device, split into hot (fp8 + per-row scale) and cold (INT4 records in the
split layout), and optionally given random-init low-rank predictors (the
``nn.Linear`` default init, U(-1/sqrt(fan_in), 1/sqrt(fan_in)) for weights and
bias).  ``records_from_rows`` is the device twin of ``format.build_records``
(the same fp32 absmax / divide / round-half-even / fp16-scale arithmetic) so
that a 32-layer cold store can be built in HBM in seconds; the two are checked
byte-for-byte against each other.
"""
from __future__ import annotations

import math

import torch

from . import format as fmt
from .hot import HotWeights
from .predictor import NeuronPredictor

H = fmt.HIDDEN_DIM


def quantize_int4_rows_torch(w: torch.Tensor):
    """(n, H) fp32 -> (packed uint8 (n, H/2), scales fp32 (n, H/128))."""
    n = w.shape[0]
    g = w.float().reshape(n, -1, fmt.GROUP_SIZE)
    s = g.abs().amax(dim=2).clamp(min=1e-8) / 7.0
    q = (g / s[:, :, None]).round().clamp(-8, 7).to(torch.int8).reshape(n, -1)
    u = (q & 0x0F).to(torch.uint8)
    packed = u[:, 0::2] | (u[:, 1::2] << 4)
    return packed, s


def records_from_rows(nids: torch.Tensor, gate: torch.Tensor, up: torch.Tensor,
                      down_cols: torch.Tensor) -> torch.Tensor:
    """(n, 6400) uint8 records on the rows' device (splitter.py:234-247)."""
    n = gate.shape[0]
    dev = gate.device
    rec = torch.zeros((n, fmt.NEURON_RECORD_BYTES), dtype=torch.uint8, device=dev)
    nids = nids.to(device=dev, dtype=torch.int64)
    rec[:, 0] = (nids & 0xFF).to(torch.uint8)
    rec[:, 1] = ((nids >> 8) & 0xFF).to(torch.uint8)
    for off, soff, w in ((fmt.OFF_GATE, fmt.OFF_GATE_SCALES, gate), (fmt.OFF_UP, fmt.OFF_UP_SCALES, up),
                         (fmt.OFF_DOWN, fmt.OFF_DOWN_SCALES, down_cols)):
        p, s = quantize_int4_rows_torch(w)
        rec[:, off:off + fmt.VEC_BYTES] = p
        rec[:, soff:soff + fmt.SCALE_BYTES_PER_VEC] = s.to(torch.float16).view(torch.uint8)
    return rec


def random_predictor(gen: torch.Generator, inter: int, rank: int = 64, dtype=torch.bfloat16,
                     device="cuda") -> NeuronPredictor:
    """NeuronPredictor with nn.Linear's default init (predictor.py:67-68)."""
    b1 = 1.0 / math.sqrt(H)
    b2 = 1.0 / math.sqrt(rank)
    down = (torch.rand((rank, H), generator=gen, device=device) * 2 - 1) * b1
    up = (torch.rand((inter, rank), generator=gen, device=device) * 2 - 1) * b2
    bias = (torch.rand((inter,), generator=gen, device=device) * 2 - 1) * b2
    return NeuronPredictor(down.to(dtype), up.to(dtype), bias.to(dtype))


class SyntheticLayer:
    """One FFN layer: dense fp32 weights (kept only when asked), its hot part,
    its cold records and LUT, norm weight and predictor."""

    def __init__(self, gen, inter, n_hot, std=0.02, device="cuda", keep_dense=False,
                 hot_ids=None, gate_bias_shift=0.0, with_predictor=False, pred_rank=64,
                 pred_dtype=torch.bfloat16, norm_jitter=0.05, per_row_scale=True):
        dev = torch.device(device)
        gate = torch.randn((inter, H), generator=gen, device=dev) * std
        up = torch.randn((inter, H), generator=gen, device=dev) * std
        down = torch.randn((H, inter), generator=gen, device=dev) * std
        if hot_ids is None:
            perm = torch.randperm(inter, generator=gen, device=dev)
            hot_ids = perm[:n_hot].sort().values
        hot_ids = hot_ids.to(dev)
        mask = torch.zeros(inter, dtype=torch.bool, device=dev)
        mask[hot_ids] = True
        cold_ids = (~mask).nonzero().flatten()
        self.inter = inter
        self.hot_ids = hot_ids
        self.cold_ids = cold_ids
        gb = None
        if gate_bias_shift:
            gb = torch.full((inter,), float(gate_bias_shift), device=dev)
        self.gate_bias = gb
        self.hot = HotWeights.from_dense(hot_ids, gate[hot_ids], up[hot_ids], down[:, hot_ids],
                                         per_row_scale=per_row_scale,
                                         gate_bias=None if gb is None else gb[hot_ids])
        self.records = records_from_rows(cold_ids, gate[cold_ids], up[cold_ids],
                                         down[:, cold_ids].t().contiguous())
        lut = torch.full((inter,), -1, dtype=torch.int32, device=dev)
        lut[cold_ids] = torch.arange(cold_ids.numel(), dtype=torch.int32, device=dev)
        self.lut = lut
        self.cold_gate_bias = None if gb is None else gb[cold_ids].contiguous()
        self.norm_w = (1.0 + norm_jitter * torch.randn((H,), generator=gen, device=dev)).to(torch.float16)
        self.predictor = random_predictor(gen, inter, pred_rank, pred_dtype, dev) if with_predictor else None
        self.dense = (gate, up, down) if keep_dense else None

    def nbytes_cold(self) -> int:
        return int(self.records.numel())


def calibrate_threshold(layers, gen, frac_active: float, n_states: int = 32, eps: float = 1e-5):
    """Logit threshold at which `frac_active` of the predicted logits fire,
    over seeded N(0,1) calibration tokens normalised by each layer's norm."""
    vals = []
    for l in layers:
        if l.predictor is None:
            continue
        dev = l.norm_w.device
        x = torch.randn((n_states, H), generator=gen, device=dev)
        xn = x * torch.rsqrt((x * x).mean(1, keepdim=True) + eps) * l.norm_w.float()
        q = xn.half().to(l.predictor.dtype).float()
        logits = (q @ l.predictor.down_w.float().t()) @ l.predictor.up_w.float().t() + \
            l.predictor.up_b.float()
        vals.append(logits.flatten())
    allv = torch.cat(vals)
    k = int(round((1.0 - frac_active) * (allv.numel() - 1)))
    return float(allv.kthvalue(k + 1).values.item())


def build_decode_stack(seed: int, dev, n_layers: int = 32, inter: int = 14336, n_hot: int = 3584,
                       rank: int = 64, active_frac: float = 0.05, eps: float = 1e-5,
                       records_on=None):
    """The 32-layer decode workload: ``n_layers`` seeded SwiGLU layers of
    4096 x ``inter`` (N(0, 0.02) weights, ``n_hot`` hot fp8 neurons, the rest
    INT4 records), each with a random-init bf16 rank-``rank`` predictor, the
    logit threshold calibrated so ``active_frac`` of the neurons are predicted
    active.  ``records_on`` maps each layer's device records to where the stack
    reads them (e.g. pinned host copies); None keeps them in HBM.  Returns
    (layers, stack, threshold logit, generator)."""
    from .stack import DecodeStack, StackLayer
    g = torch.Generator(device=dev).manual_seed(seed)
    layers = [SyntheticLayer(g, inter, n_hot, std=0.02, device=dev, with_predictor=True,
                             pred_rank=rank, pred_dtype=torch.bfloat16) for _ in range(n_layers)]
    thr = calibrate_threshold(layers, g, active_frac, eps=eps)
    recs = [records_on(l.records) if records_on is not None else l.records for l in layers]
    st = DecodeStack([StackLayer(l.hot, r, l.lut, l.norm_w, l.predictor)
                      for l, r in zip(layers, recs)], inter, eps, "silu", False, thr)
    # size the cold pass for the calibrated active fraction with headroom
    st.set_expected_active(int(1.3 * active_frac * (inter - n_hot)))
    return layers, st, thr, g


def zipf_layers(gen, n_layers: int, inter: int = 14336, hot_frac: float = 0.2, s: float = 1.1,
                cold_active: float = 0.15, batch: int = 8, eps: float = 1e-5, device="cuda",
                n_cal: int = 64, std: float = 0.02):
    """Layers whose neuron firing popularity is Zipf(s) over the intermediate
    dimension: each layer draws a random rank for every neuron; the top
    ``hot_frac`` by rank are hot (fp8), the rest cold (INT4 records); the
    random-init bf16 predictor's bias is set so that a neuron of rank r is
    predicted active with probability a_r = min(0.95, K (r + 1)^-s) for the
    batch-mean query of ``batch`` N(0, 1) tokens (engine.py:277), K chosen so
    that ``cold_active`` of the cold neurons fire on average.  The bias is
    b = -mu + sigma * Phi^-1(a) from the per-neuron mean mu and spread sigma
    of the bias-free logits over ``n_cal`` seeded calibration batches, for the
    threshold p = 0.5 (logit 0).  Returns the layers."""
    dev = torch.device(device)
    n_hot = int(round(hot_frac * inter))
    layers = []
    for _ in range(n_layers):
        rank = torch.randperm(inter, generator=gen, device=dev)          # rank of each neuron
        hot_ids = (rank < n_hot).nonzero().flatten().sort().values
        lay = SyntheticLayer(gen, inter, n_hot, std=std, device=dev, hot_ids=hot_ids,
                             with_predictor=True, pred_dtype=torch.bfloat16)
        p = lay.predictor
        # target activation probability by rank; K by bisection on the cold mean
        r = rank.double() + 1.0
        cold = rank >= n_hot
        lo, hi = 0.0, 1e6
        for _ in range(80):
            K = 0.5 * (lo + hi)
            a = torch.clamp(K * r.pow(-s), max=0.95)
            if a[cold].mean().item() < cold_active:
                lo = K
            else:
                hi = K
        a = torch.clamp(0.5 * (lo + hi) * r.pow(-s), min=1e-6, max=0.95)
        # bias-free logits of calibration batch-mean queries
        x = torch.randn((n_cal, batch, H), generator=gen, device=dev)
        xn = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * lay.norm_w.float()
        q = xn.half().float().mean(1).half().to(torch.bfloat16).float()
        z = (q @ p.down_w.float().t()) @ p.up_w.float().t()
        mu, sigma = z.mean(0).double(), z.std(0).double().clamp(min=1e-6)
        b = -mu + sigma * torch.special.ndtri(a)
        p.up_b = b.to(p.dtype).contiguous()
        lay.zipf_rank = rank
        layers.append(lay)
    return layers
