"""Multi-token FFN (batch decode with a shared active set, prefill chunks) on
the MFMA path, through oi2_ffn_forward with batch >= 2, against the float64
oracle over the same quantised weights.  Bar: max rel err <= 1e-2 and cosine
>= 0.9999 per checked row set."""
import math

import numpy as np
import pytest
import torch

from oi2.layer import ColdNeurons, _ffn
from oi2.store import ColdSection
from oi2.synth import SyntheticLayer
from oracle import oracle as O
from tests.gpu_helpers import EPS, assert_ffn_close, cold_dense, hot_dense, normed_f16

pytestmark = pytest.mark.gpu
H = 4096


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


def _section(lay):
    return ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut, lay.lut.cpu().numpy(),
                       lay.inter)


@pytest.fixture(scope="module")
def layer25(dev):
    g = torch.Generator(device=dev).manual_seed(31)
    return SyntheticLayer(g, 14336, 3584, device=dev), g


@pytest.mark.parametrize("B", [2, 8, 17, 64])
def test_batch_decode_shared_active_set(dev, layer25, B):
    lay, g = layer25
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[: int(0.15 * n_cold)].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((B, H), generator=g, device=dev).half()
    out, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, add_residual=True,
                    want_y32=True)
    torch.cuda.synchronize()
    rows = list(range(B)) if B <= 8 else sorted({0, 1, B // 2, B - 2, B - 1})
    assert max(rows) < B
    xn = normed_f16(x[rows], lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    Gc, Uc, Dc = cold_dense(lay.records, slots)
    ref = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
    y = y32[rows].cpu().numpy()
    for r in range(len(rows)):
        assert_ffn_close(y[r], ref[r], what=f"B={B} row {rows[r]}")
    assert_ffn_close(out[rows].float().cpu().numpy(), x[rows].float().cpu().numpy() + ref,
                     tol=2e-3, cos_min=0.99999, what="residual out")
    # every row of the batch equals the same token run alone (decode path)
    one = _ffn(x[rows[-1]:rows[-1] + 1], lay.norm_w, EPS, lay.hot, cold, "silu", False, True,
               want_y32=True)[1]
    assert_ffn_close(y32[rows[-1]].cpu().numpy(), one[0].cpu().numpy(), tol=2e-3, cos_min=0.99999,
                     what="batch row vs single token")


@pytest.fixture(scope="module")
def chain3(dev):
    """Three layers of 4096 x 14336 (3584 hot), each with 30 % of its cold
    records active."""
    g = torch.Generator(device=dev).manual_seed(77)
    lays, colds = [], []
    for _ in range(3):
        lay = SyntheticLayer(g, 14336, 3584, device=dev)
        n = lay.records.shape[0]
        slots = torch.randperm(n, generator=g, device=dev)[: int(0.3 * n)].int()
        lays.append(lay)
        colds.append(ColdNeurons.from_slots(_section(lay), slots))
    return lays, colds, g


@pytest.mark.parametrize("B", [8, 40, 64, 512])
def test_batch_chain_equals_separate_calls(dev, chain3, B):
    """Three layers through oi2_ffn_forward_chain (each call takes the
    previous call's normalised rows and writes the next layer's) give the
    same bits as three oi2_ffn_forward calls with their own norms, and every
    xn_next equals oi2_rmsnorm of that call's output bit for bit."""
    from oi2.layer import rmsnorm
    lays, colds, g = chain3
    x0 = torch.randn((B, H), generator=g, device=dev).half()
    ref, x = [], x0
    for lay, c in zip(lays, colds):
        x = _ffn(x, lay.norm_w, EPS, lay.hot, c, "silu", False, True)
        ref.append(x)
    x, xn = x0, None
    for i, (lay, c) in enumerate(zip(lays, colds)):
        nxt = lays[i + 1].norm_w if i + 1 < len(lays) else None
        r = _ffn(x, lay.norm_w, EPS, lay.hot, c, "silu", False, True, xn_in=xn, next_norm_w=nxt)
        x, xn = r if nxt is not None else (r, None)
        torch.cuda.synchronize()
        assert torch.equal(x, ref[i]), f"B={B} layer {i}"
        if nxt is not None:
            assert torch.equal(xn, rmsnorm(x, nxt, EPS)), f"B={B} layer {i} xn_next"


@pytest.mark.parametrize("B", [3, 8, 16])
def test_batch_cold_only_small(dev, layer25, B):
    """Up to 16 tokens with no hot half: the cold down's ranges are added by
    the final launch, with the residual."""
    lay, g = layer25
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[: int(0.15 * n_cold)].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((B, H), generator=g, device=dev).half()
    out, y32 = _ffn(x, lay.norm_w, EPS, None, cold, "silu", False, add_residual=True, want_y32=True)
    torch.cuda.synchronize()
    xn = normed_f16(x, lay.norm_w)
    Gc, Uc, Dc = cold_dense(lay.records, slots)
    ref = O.sparse_ffn(xn, "silu", False, None, None, None, Gc, Uc, Dc)
    y = y32.cpu().numpy()
    for r in range(B):
        assert_ffn_close(y[r], ref[r], what=f"cold only B={B} row {r}")
    assert_ffn_close(out.float().cpu().numpy(), x.float().cpu().numpy() + ref, tol=2e-3, cos_min=0.99999,
                     what="cold only residual out")


@pytest.mark.parametrize("B,frac", [(64, 0.5), (40, 1.0), (33, 0.47)])
def test_batch_wide_tiles(dev, layer25, B, frac):
    """At most 64 tokens with more 32-neuron units than the GPU has CUs: part
    of the gate/up tiles are two units wide (list items at 0.5 and 0.47, the
    last tile part full at 0.47; every item and some hot rows at 1.0).  Rows
    against the float64 oracle, every row against float32 torch over the same
    dequantised weights."""
    lay, g = layer25
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[: int(frac * n_cold)].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((B, H), generator=g, device=dev).half()
    _, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, False, want_y32=True)
    torch.cuda.synchronize()
    xn = normed_f16(x, lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    Gc, Uc, Dc = cold_dense(lay.records, slots)
    rows = sorted({0, 1, 31, 32, B // 2, B - 1})
    ref = O.sparse_ffn(xn[rows], "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
    y = y32.cpu().numpy()
    for k, r in enumerate(rows):
        assert_ffn_close(y[r], ref[k], what=f"B={B} frac={frac} row {r}")
    f32 = lambda a: torch.as_tensor(a, dtype=torch.float32, device=dev)
    xa = f32(xn)
    silu = torch.nn.functional.silu
    hh = silu(xa @ f32(Gh).T) * (xa @ f32(Uh).T)
    hc = silu(xa @ f32(Gc).T) * (xa @ f32(Uc).T)
    ref_all = (hh @ f32(Dh).T + hc @ f32(Dc).T).double().cpu().numpy()
    assert_ffn_close(y, ref_all, what=f"B={B} frac={frac} all rows")


@pytest.fixture(scope="module")
def drelu_layer(dev):
    """Config 2's layer: dReLU at 4096 x 14336, 25 % hot, gate pre-activation
    shifted by -1.3 sigma so that ~10 % of gates are positive."""
    g = torch.Generator(device=dev).manual_seed(22)
    sigma = 0.02 * math.sqrt(H)
    lay = SyntheticLayer(g, 14336, 3584, device=dev, gate_bias_shift=-1.3 * sigma)
    dense = cold_dense(lay.records, np.arange(lay.records.shape[0]))
    return lay, g, dense


@pytest.mark.parametrize("B", [16, 64, 512])
def test_batch_drelu_union_of_firing_sets_equals_dense(dev, drelu_layer, B):
    """B independent dReLU tokens with a gate bias over the union of their
    true firing sets: a neuron outside a token's set contributes exactly zero
    to it, so the union reproduces each token's dense FFN.  B = 64 is survey
    config 2; 16 runs the skinny small-batch kernels, 64 the 64-token tiles,
    512 the prefill tiles (relu epilogues with the bias on each).  Rows spread
    over the batch against the float64 oracle; for B >= 64 every row against a
    float32 torch reference over the same dequantised weights."""
    lay, g, (Gc_all, Uc_all, Dc_all) = drelu_layer
    inter = lay.inter
    x = torch.randn((B, H), generator=g, device=dev).half()
    xn = normed_f16(x, lay.norm_w)
    bc = lay.cold_gate_bias.cpu().numpy().astype(np.float64)
    fire = (np.maximum(xn @ Gc_all.T + bc, 0) * np.maximum(xn @ Uc_all.T, 0)) != 0
    per_token = fire.sum(axis=1) / Gc_all.shape[0]
    assert 0.02 < per_token.mean() < 0.08          # ~4.8 % of cold neurons fire per token
    union = np.nonzero(fire.any(axis=0))[0]
    assert 0.2 * inter < union.size < 0.8 * inter
    cold = ColdNeurons.from_slots(_section(lay), union, gate_bias=lay.cold_gate_bias)
    _, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "relu", True, False, want_y32=True)
    torch.cuda.synchronize()
    Gh, Uh, Dh = hot_dense(lay.hot)
    bh = lay.hot.gate_bias.cpu().numpy().astype(np.float64)
    rows = list(range(B)) if B <= 16 else sorted({0, 1, 31, 63, B // 2, B - 2, B - 1})
    assert max(rows) < B
    dense = O.sparse_ffn(xn[rows], "relu", True, Gh, Uh, Dh, Gc_all, Uc_all, Dc_all, bh, bc)
    y = y32.cpu().numpy()
    for k, r in enumerate(rows):
        assert_ffn_close(y[r], dense[k], what=f"dReLU B={B} row {r}")
    if B >= 64:
        f32 = lambda a: torch.as_tensor(a, dtype=torch.float32, device=dev)
        xa = f32(xn)
        relu = torch.nn.functional.relu
        hh = relu(xa @ f32(Gh).T + f32(bh)) * relu(xa @ f32(Uh).T)
        hc = relu(xa @ f32(Gc_all).T + f32(bc)) * relu(xa @ f32(Uc_all).T)
        ref_all = (hh @ f32(Dh).T + hc @ f32(Dc_all).T).double().cpu().numpy()
        assert_ffn_close(y, ref_all, what=f"dReLU B={B} all rows")


@pytest.mark.parametrize("B", [70, 159, 160, 200, 400])
def test_batch_edge_shapes(dev, B):
    """Token count not a multiple of the 64- or 128-row tile (70 and 159 on
    the 64-token tiles, 160, 200 and 400 on the prefill tiles), n_hot not a multiple
    of the 128 K block, a chunked active list with an empty chunk, duplicates
    and invalid slots, one half missing."""
    g = torch.Generator(device=dev).manual_seed(6)
    lay = SyntheticLayer(g, 2000, 1000, device=dev)
    sec = _section(lay)
    x = torch.randn((B, H), generator=g, device=dev).half()
    rows = sorted({0, 5, 63, 64, B // 2, B - 2, B - 1})
    assert max(rows) < B
    xn = normed_f16(x[rows], lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    sl = torch.full((3 * 40,), -7, dtype=torch.int32, device=dev)
    sl[0:37] = torch.arange(37, dtype=torch.int32) * 3
    sl[80:93] = torch.tensor([5, 5, 900, -1, 10 ** 6, 17, 999, 998, 1, 2, 3, 4, 700],
                             dtype=torch.int32)
    counts = torch.tensor([37, 0, 13], dtype=torch.int32, device=dev)
    cold = ColdNeurons(sec, sl, counts, 3, 40)
    valid = [s for s in sl[0:37].tolist() + sl[80:93].tolist() if 0 <= s < lay.records.shape[0]]
    Gc, Uc, Dc = cold_dense(lay.records, valid)
    for hot, c, what in ((lay.hot, cold, "both"), (None, cold, "cold only"),
                         (lay.hot, None, "hot only")):
        _, y32 = _ffn(x, lay.norm_w, EPS, hot, c, "silu", False, False, want_y32=True)
        ref = O.sparse_ffn(xn, "silu", False, *(hot_dense(hot) if hot is not None else
                                                  (None, None, None)),
                           *((Gc, Uc, Dc) if c is not None else (None, None, None)))
        y = y32[rows].cpu().numpy()
        for r in range(len(rows)):
            assert_ffn_close(y[r], ref[r], what=f"{what} row {rows[r]}")
    # both halves empty: zeros
    _, y32 = _ffn(x[:3], lay.norm_w, EPS, None, None, "silu", False, False, want_y32=True)
    assert torch.count_nonzero(y32) == 0


def test_prefill_chunk_512(dev):
    """A 512-token prefill chunk (survey config 5 geometry, one layer): hot
    fp8 dense product plus the chunk's union of cold neurons (40 %).  Oracle
    rows spread over every 64-row tile; all rows against a float32 torch
    reference over the same dequantised weights."""
    g = torch.Generator(device=dev).manual_seed(51)
    lay = SyntheticLayer(g, 14336, 3584, device=dev)
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[: int(0.4 * n_cold)].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    M = 512
    x = torch.randn((M, H), generator=g, device=dev).to(torch.bfloat16).half()
    out, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, True, want_y32=True)
    torch.cuda.synchronize()
    rows = [0, 70, 141, 200, 255, 300, 383, 447, 511]
    xn = normed_f16(x[rows], lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    Gc, Uc, Dc = cold_dense(lay.records, slots)
    ref = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
    y = y32[rows].cpu().numpy()
    for r in range(len(rows)):
        assert_ffn_close(y[r], ref[r], what=f"prefill row {rows[r]}")
    # all 512 rows: float32 torch over the dequantised weights
    f32 = lambda a: torch.as_tensor(a, dtype=torch.float32, device=dev)
    xn_all = torch.as_tensor(normed_f16(x, lay.norm_w), dtype=torch.float32, device=dev)
    hh = torch.nn.functional.silu(xn_all @ f32(Gh).T) * (xn_all @ f32(Uh).T)
    hc = torch.nn.functional.silu(xn_all @ f32(Gc).T) * (xn_all @ f32(Uc).T)
    ref_all = (hh @ f32(Dh).T + hc @ f32(Dc).T).double().cpu().numpy()
    assert_ffn_close(y32.cpu().numpy(), ref_all, what="prefill all rows")


def test_prefill_chain_32_layers(dev):
    """Survey config 5 end to end: a 512-token chunk through 32 layers
    (engine.py:424-438's chain: RMSNorm in front of every FFN, the residual
    carried), each layer with its own 40 % cold union.  Teacher-forced on the
    GPU's own layer inputs, layers 0 and 31 match the float64 oracle on rows
    spread over the tiles and float32 torch on every row; every layer's
    output is finite and its residual update within the FFN bar of a float32
    reference over the same weights on the first, middle and last layers."""
    g = torch.Generator(device=dev).manual_seed(61)
    n_layers, M = 32, 512
    layers, colds, slot_sets = [], [], []
    for _ in range(n_layers):
        lay = SyntheticLayer(g, 14336, 3584, device=dev)
        n_cold = lay.records.shape[0]
        slots = torch.randperm(n_cold, generator=g, device=dev)[: int(0.4 * n_cold)].int()
        layers.append(lay)
        slot_sets.append(slots)
        colds.append(ColdNeurons.from_slots(_section(lay), slots))
    x = torch.randn((M, H), generator=g, device=dev).to(torch.bfloat16).half()
    ins, outs = [], []
    for lay, cold in zip(layers, colds):
        ins.append(x)
        x = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, True)
        outs.append(x)
    torch.cuda.synchronize()
    for o in outs:
        assert torch.isfinite(o.float()).all()
    f32 = lambda a: torch.as_tensor(a, dtype=torch.float32, device=dev)
    rows = [0, 77, 190, 256, 383, 511]
    for L in (0, 15, 31):
        lay = layers[L]
        Gh, Uh, Dh = hot_dense(lay.hot)
        Gc, Uc, Dc = cold_dense(lay.records, slot_sets[L])
        xn_all = torch.as_tensor(normed_f16(ins[L], lay.norm_w), dtype=torch.float32, device=dev)
        hh = torch.nn.functional.silu(xn_all @ f32(Gh).T) * (xn_all @ f32(Uh).T)
        hc = torch.nn.functional.silu(xn_all @ f32(Gc).T) * (xn_all @ f32(Uc).T)
        ref_all = (hh @ f32(Dh).T + hc @ f32(Dc).T).double().cpu().numpy()
        upd = outs[L].double().cpu().numpy() - ins[L].double().cpu().numpy()
        # the output is fp16(x + y): the update carries one fp16 rounding of x + y
        assert_ffn_close(upd, ref_all, tol=2e-2, cos_min=0.9999, what=f"layer {L} update, all rows")
        if L in (0, 31):
            _, y32 = _ffn(ins[L], lay.norm_w, EPS, lay.hot, colds[L], "silu", False, True, want_y32=True)
            torch.cuda.synchronize()
            xn = normed_f16(ins[L][rows], lay.norm_w)
            ref = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
            y = y32[rows].cpu().numpy()
            for k, r in enumerate(rows):
                assert_ffn_close(y[k], ref[k], what=f"layer {L} row {r} vs oracle")
            assert_ffn_close(y32.cpu().numpy(), ref_all, what=f"layer {L} all rows")


@pytest.mark.parametrize("B", [3, 17, 96, 300])
def test_batch_ignores_workspace_contents(dev, layer25, B):
    """The workspace is scratch: filled with NaN before the call (every byte
    0xFF), the result is the same as with a zeroed one.  Covers the columns
    past the active list's end, which no gate/up kernel writes."""
    from oi2.layer import workspace_bytes
    lay, g = layer25
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[:1001].int()   # not a tile multiple
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((B, H), generator=g, device=dev).half()
    nbytes = workspace_bytes(B, lay.hot, cold)
    outs = []
    for fill in (0xFF, 0x00):
        ws = torch.full((nbytes,), fill, dtype=torch.uint8, device=dev)
        outs.append(_ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, True, want_y32=True,
                         workspace=ws)[1].cpu().numpy())
    assert np.isfinite(outs[0]).all()
    assert_ffn_close(outs[0].reshape(-1), outs[1].reshape(-1), tol=1e-5, cos_min=0.999999,
                     what=f"B={B} NaN-filled vs zeroed workspace")


@pytest.mark.parametrize("B", [2, 8, 16, 17, 64, 200, 512])
def test_batch_is_bit_reproducible(dev, layer25, B):
    """No batch kernel accumulates with atomics: up to 16 tokens the cold
    down's item ranges are added in range order, from 17 tokens every down
    workgroup's partial sum is added in range order by the final launch, so
    repeated calls (the workspace NaN-filled in between, and only the hot
    half or only the cold half too) give the same bits."""
    from oi2.layer import workspace_bytes
    lay, g = layer25
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[:1613].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((B, H), generator=g, device=dev).half()
    for hot, cd, what in ((lay.hot, cold, "hot + cold"), (None, cold, "cold only"), (lay.hot, None, "hot only")):
        nbytes = workspace_bytes(B, hot, cd)
        runs = []
        for fill in (0xFF, 0x00, 0x5A):
            ws = torch.full((nbytes,), fill, dtype=torch.uint8, device=dev)
            out, y32 = _ffn(x, lay.norm_w, EPS, hot, cd, "silu", False, True, want_y32=True, workspace=ws)
            runs.append((out.clone(), y32.clone()))
        torch.cuda.synchronize()
        print(f"[batch] B={B} {what}: {len(runs)} runs", flush=True)
        for out, y32 in runs[1:]:
            assert torch.equal(out, runs[0][0]) and torch.equal(y32, runs[0][1]), f"B={B} {what}"
        if hot is None:
            Gc, Uc, Dc = cold_dense(lay.records, slots)
            ref = O.sparse_ffn(normed_f16(x, lay.norm_w), "silu", False, None, None, None, Gc, Uc, Dc)
            assert_ffn_close(runs[0][1].cpu().numpy(), ref, what=f"B={B} cold only against the oracle")
