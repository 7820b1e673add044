"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars: bit-exact for dequant, fp8 decode and index sets (outside the 1e-6
logit band); FFN outputs within max rel err 1e-2 and cosine >= 0.9999 of the
float64 oracle over the same quantised weights.
"""
import math
import os
import tempfile
import hashlib
import json

import numpy as np
import pytest
import torch

import oi2
from oi2 import _lib
from oi2.layer import ColdNeurons, _ffn, rmsnorm
from oi2.store import ColdSection
from oi2.synth import SyntheticLayer, calibrate_threshold, random_predictor, records_from_rows
from oracle import oracle as O
from tests.fixtures import synthetic_cold_file
from tests.gpu_helpers import (EPS, assert_ffn_close, chunked_ids, cold_dense, hot_dense,
                               normed_f16, pred_weights, query_for)

pytestmark = pytest.mark.gpu
H = 4096
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


def _section(lay):
    return ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut, lay.lut.cpu().numpy(),
                       lay.inter)


# ── FP8 decode through the hot GEMV ──────────────────────────────────────────

def test_fp8_decode_table_exact(dev):
    """Hot neuron k's gate row holds code k at position 0; x = +-e_0, up = 1,
    down = identity, relu(g)*u: y_k is the decoded code exactly."""
    codes = np.arange(256, dtype=np.uint8)
    codes[[0x7F, 0xFF]] = 0                      # the two NaN codes
    n = 256
    gate = torch.zeros((n, H), dtype=torch.uint8)
    gate[:, 0] = torch.from_numpy(codes)
    up = torch.zeros((n, H), dtype=torch.uint8)
    up[:, 0] = 0x38                               # 1.0
    down = torch.zeros((H, n), dtype=torch.uint8)
    down[torch.arange(n), torch.arange(n)] = 0x38
    ones_n = torch.ones(n)
    hot = oi2.HotWeights(torch.arange(n), gate.to(dev), up.to(dev), down.to(dev), ones_n.to(dev),
                         ones_n.to(dev), torch.ones(H).to(dev))
    table = O.FP8_TABLE.copy()
    table[[0x7F, 0xFF]] = 0.0
    for sign in (1.0, -1.0):
        x = torch.zeros((1, H), dtype=torch.float16, device=dev)
        x[0, 0] = sign
        _, y = _ffn(x, None, 0.0, hot, None, "relu", False, add_residual=False, want_y32=True)
        got = y[0, :n].double().cpu().numpy()
        want = sign * np.maximum(sign * table, 0.0)
        assert np.array_equal(got, want), np.nonzero(got != want)


# ── INT4 record dequant ──────────────────────────────────────────────────────

def test_dequant_records_bit_exact(dev):
    g = torch.Generator(device=dev).manual_seed(2)
    n = 300
    rows = [torch.randn((n, H), generator=g, device=dev) * s for s in (0.02, 1.0, 5.0)]
    rec = records_from_rows(torch.arange(n), *rows)
    # one record of raw bytes: every byte value, every scale sign
    rec[7, 2:6146] = torch.arange(6144, device=dev).to(torch.uint8)
    rec[7, 6146:6338] = torch.tensor(np.array([0.5, -1.25, 3.0, 2.0 ** -14] * 24, np.float16)
                                     .view(np.uint8)).to(dev)
    slots = torch.tensor([7, 0, 299, 7, 150, 3], dtype=torch.int32, device=dev)
    out = torch.empty((3, 6, H), device=dev)
    down_t = torch.empty((H, 6), device=dev)
    L = _lib.lib()
    _lib.check(L.oi2_dequant_records(rec.data_ptr(), n, slots.data_ptr(), 6, out[0].data_ptr(),
                                     out[1].data_ptr(), down_t.data_ptr(), None))
    torch.cuda.synchronize()
    G, U, D = O.records_to_dense(rec.cpu().numpy(), slots.cpu().numpy())
    assert np.array_equal(out[0].cpu().numpy().astype(np.float64), G)
    assert np.array_equal(out[1].cpu().numpy().astype(np.float64), U)
    assert np.array_equal(down_t.cpu().numpy().astype(np.float64), D)


def test_store_read_neurons_matches_reference_truth(dev):
    """tests/test_cold_store.py:28-91 semantics on the reference fixture's
    byte image, values hashed against the reference's own dequant output."""
    golden = json.load(open(os.path.join(GOLDEN, "cold_seed0.json")))
    with tempfile.TemporaryDirectory() as tmp:
        cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp, 4, 16, 0)
        store = oi2.ColdWeightStore(cold_bin, cold_idx, config, device=dev)
        try:
            for li in range(4):
                nids = layers[li][0]
                for nid in nids:
                    gate, up, down = store.read_neurons(li, 0, [nid])
                    assert gate.shape == (1, H) and up.shape == (1, H) and down.shape == (H, 1)
                    for name, v in (("gate", gate[0]), ("up", up[0]), ("down", down[:, 0])):
                        h = hashlib.sha256(v.cpu().numpy().astype("<f4").tobytes()).hexdigest()
                        assert h == golden["truth_sha256"][f"{li}:{nid}:{name}"]
            ids0 = layers[0][0]
            out = store.read_neurons(0, 0, sorted(ids0))
            assert out[0].shape == (16, H) and out[2].shape == (H, 16)
            first = store.read_neurons(0, 0, [sorted(ids0)[0]])
            assert torch.equal(out[0][0], first[0][0])
            absent = max(ids0) + 1000
            mixed = store.read_neurons(0, 0, [ids0[0], absent, ids0[0]])
            assert mixed[0].shape[0] == 2 and torch.equal(mixed[0][0], mixed[0][1])
            assert store.read_neurons(0, 0, [absent, absent + 1]) is None
            again = store.read_neurons(1, 0, layers[1][0][:4])
            assert (1, 0) in store._offset_cache
            for a, b in zip(again, store.read_neurons(1, 0, layers[1][0][:4])):
                assert torch.equal(a, b)
            # records in pinned host memory, decoded over PCIe: same bits
            pstore = oi2.ColdWeightStore(cold_bin, cold_idx, config, device=dev, pinned=True)
            try:
                for li in range(4):
                    assert pstore.section(li).records.is_pinned()
                    req = layers[li][0][::-1] + [absent]
                    for a, b in zip(pstore.read_neurons(li, 0, req), store.read_neurons(li, 0, req)):
                        assert a.device == b.device and torch.equal(a, b)
            finally:
                pstore.close()
        finally:
            store.close()


# ── the fused FFN ────────────────────────────────────────────────────────────

@pytest.fixture(scope="module")
def layer_swiglu(dev):
    """Single SwiGLU layer 4096 x 14336, 20 % hot (2867) fp8 with per-row
    scales, the rest INT4 records."""
    g = torch.Generator(device=dev).manual_seed(11)
    lay = SyntheticLayer(g, 14336, 2867, device=dev)
    return lay, g


def test_ffn_swiglu_full_geometry(dev, layer_swiglu):
    lay, g = layer_swiglu
    n_cold = lay.records.shape[0]
    slots = torch.randperm(n_cold, generator=g, device=dev)[: n_cold // 10].int()
    cold = ColdNeurons.from_slots(_section(lay), slots)
    x = torch.randn((1, H), generator=g, device=dev).half()
    out, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, add_residual=True,
                    want_y32=True)
    torch.cuda.synchronize()
    xn = normed_f16(x, lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    Gc, Uc, Dc = cold_dense(lay.records, slots)
    ref = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
    assert_ffn_close(y32.cpu().numpy(), ref, what="y32")
    assert_ffn_close(out.float().cpu().numpy(), x.float().cpu().numpy() + ref, tol=2e-3,
                     cos_min=0.99999, what="residual out")
    # each half on its own
    _, yh = _ffn(x, lay.norm_w, EPS, lay.hot, None, "silu", False, False, want_y32=True)
    _, yc = _ffn(x, lay.norm_w, EPS, None, cold, "silu", False, False, want_y32=True)
    assert_ffn_close(yh.cpu().numpy(), O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, None, None, None),
                     what="hot half")
    assert_ffn_close(yc.cpu().numpy(), O.sparse_ffn(xn, "silu", False, None, None, None, Gc, Uc, Dc),
                     what="cold half")


def test_ffn_drelu_true_firing_set_equals_dense(dev):
    """dReLU with a -1.3 sigma gate shift: hot + the truly firing cold
    neurons equals the FFN over every neuron (non-firing terms are zero)."""
    g = torch.Generator(device=dev).manual_seed(21)
    inter = 14336
    sigma = 0.02 * math.sqrt(H)
    lay = SyntheticLayer(g, inter, 3584, device=dev, gate_bias_shift=-1.3 * sigma)
    x = torch.randn((1, H), generator=g, device=dev).half()
    xn = normed_f16(x, lay.norm_w)
    Gc_all, Uc_all, Dc_all = cold_dense(lay.records, np.arange(lay.records.shape[0]))
    bc = lay.cold_gate_bias.cpu().numpy().astype(np.float64)
    gc = xn @ Gc_all.T + bc
    uc = xn @ Uc_all.T
    firing = np.nonzero((np.maximum(gc, 0) * np.maximum(uc, 0)).ravel() != 0)[0]
    assert 0.01 * inter < firing.size < 0.15 * inter
    cold = ColdNeurons.from_slots(_section(lay), firing, gate_bias=lay.cold_gate_bias)
    _, y32 = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "relu", True, False, want_y32=True)
    Gh, Uh, Dh = hot_dense(lay.hot)
    bh = lay.hot.gate_bias.cpu().numpy().astype(np.float64)
    dense = O.sparse_ffn(xn, "relu", True, Gh, Uh, Dh, Gc_all, Uc_all, Dc_all, bh, bc)
    assert_ffn_close(y32.cpu().numpy(), dense, what="dReLU vs dense")


def test_ffn_edge_cases(dev):
    g = torch.Generator(device=dev).manual_seed(5)
    lay = SyntheticLayer(g, 1000, 13, device=dev)
    sec = _section(lay)
    x = torch.randn((1, H), generator=g, device=dev).half()
    xn = normed_f16(x, lay.norm_w)
    Gh, Uh, Dh = hot_dense(lay.hot)
    # both halves empty -> zeros (engine.py:207-208)
    _, y = _ffn(x, lay.norm_w, EPS, None, None, "silu", False, False, want_y32=True)
    assert torch.count_nonzero(y) == 0
    # duplicates count twice, invalid slots are skipped
    slots = [5, 5, 900, -1, 10 ** 6, 17]
    cold = ColdNeurons.from_slots(sec, slots)
    _, y = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, False, want_y32=True)
    Gc, Uc, Dc = cold_dense(lay.records, [5, 5, 900, 17])
    assert_ffn_close(y.cpu().numpy(), O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc))
    # chunked active list with uneven counts, including an empty chunk
    sl = torch.full((3 * 8,), -7, dtype=torch.int32, device=dev)
    sl[0:3] = torch.tensor([1, 2, 3])
    sl[16:21] = torch.tensor([40, 41, 42, 43, 44])
    counts = torch.tensor([3, 0, 5], dtype=torch.int32, device=dev)
    chunked = ColdNeurons(sec, sl, counts, 3, 8)
    _, y = _ffn(x, lay.norm_w, EPS, None, chunked, "silu", False, False, want_y32=True)
    Gc, Uc, Dc = cold_dense(lay.records, [1, 2, 3, 40, 41, 42, 43, 44])
    assert_ffn_close(y.cpu().numpy(), O.sparse_ffn(xn, "silu", False, None, None, None, Gc, Uc, Dc))
    # batch of 3 rows shares the active set
    xb = torch.randn((3, H), generator=g, device=dev).half()
    cold = ColdNeurons.from_slots(sec, [0, 9, 33])
    _, yb = _ffn(xb, lay.norm_w, EPS, lay.hot, cold, "silu", False, False, want_y32=True)
    Gc, Uc, Dc = cold_dense(lay.records, [0, 9, 33])
    ref = O.sparse_ffn(normed_f16(xb, lay.norm_w), "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
    assert_ffn_close(yb.cpu().numpy(), ref, what="batch 3")


def test_rmsnorm_within_one_fp16_ulp(dev):
    g = torch.Generator(device=dev).manual_seed(3)
    x = (torch.randn((5, H), generator=g, device=dev) * torch.tensor([1e-2, 1, 30, 300, 3e3],
                                                                     device=dev)[:, None]).half()
    w = (1 + 0.3 * torch.randn(H, generator=g, device=dev)).half()
    got = rmsnorm(x, w, EPS).cpu().numpy()
    ref = O.rmsnorm(x.float().cpu().numpy(), w.float().cpu().numpy(), EPS)
    ulp = np.abs(np.spacing(ref.astype(np.float16))).astype(np.float64)
    assert (np.abs(got.astype(np.float64) - ref) <= ulp).all()
    assert (got == ref.astype(np.float16)).mean() > 0.99


# ── predictor ────────────────────────────────────────────────────────────────

LOGIT_BAND = 1e-6     # the contract's exemption band around the threshold


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("h_dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_predictor_logits_mask_and_selection(dev, dtype, h_dtype):
    """Logits within the 1e-6 band of the float64 oracle (the largest error is
    printed), so that the mask equals the oracle's outside that band; the
    hidden state, of any float dtype, is cast straight to the predictor dtype
    (predictor.py:455)."""
    g = torch.Generator(device=dev).manual_seed(31)
    inter = 14336
    pred = random_predictor(g, inter, 64, dtype, dev)
    D, U, b = pred_weights(pred)
    x = (torch.randn((2, H), generator=g, device=dev) * 1.7).to(h_dtype)
    logits = pred.logits(x)
    probs = pred(x)
    mask = pred.predict_mask(x, 0.5)
    torch.cuda.synchronize()
    worst = 0.0
    for r in range(2):
        q = x[r].float().cpu().numpy()
        if dtype == torch.bfloat16:
            q = O.to_bf16(q)
        ref = O.predictor_logits(q.astype(np.float64), D, U, b)
        got = logits[r].double().cpu().numpy()
        worst = max(worst, float(np.abs(got - ref).max()))
        # the sums run in double precision: the fp32 logits returned are the
        # oracle's logits rounded once (at most one fp32 ulp away)
        assert (got == ref.astype(np.float32)).mean() > 0.999
        ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
        assert (np.abs(got - ref) <= ulp).all()
        # and the mask is decided on the double logit: equal to the oracle's
        # outside a band a thousand times narrower than the contract's
        amb = O.ambiguous(ref, 0.5, band=1e-3 * LOGIT_BAND)
        assert np.array_equal(mask[r].cpu().numpy()[~amb], (ref >= 0.0)[~amb])
        assert np.allclose(probs[r].double().cpu().numpy(), 1 / (1 + np.exp(-ref)), atol=1e-6)
    print(f"predictor {dtype} <- {h_dtype}: max |fp32 logit - oracle| = {worst:.3e}")
    assert worst < LOGIT_BAND
    # on-device selection: RMSNorm -> query -> threshold -> LUT filter -> ascending
    norm_w = (1 + 0.05 * torch.randn(H, generator=g, device=dev)).half()
    hot_ids = torch.randperm(inter, generator=g, device=dev)[:3584]
    lut = torch.arange(inter, dtype=torch.int32, device=dev) * 3
    lut[hot_ids] = -1
    thr_p = 0.52
    for rows in (1, 3):
        xq = torch.randn((rows, H), generator=g, device=dev).half()
        nc = (inter + 255) // 256
        slots = torch.empty(nc * 256, dtype=torch.int32, device=dev)
        ids = torch.empty_like(slots)
        counts = torch.empty(nc, dtype=torch.int32, device=dev)
        dslots = torch.empty(inter, dtype=torch.int32, device=dev)
        dids = torch.empty_like(dslots)
        total = torch.empty(1, dtype=torch.int32, device=dev)
        p = pred.struct()
        import ctypes
        L = _lib.lib()
        wsb = L.oi2_predict_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        _lib.check(L.oi2_predict_select(xq.data_ptr(), rows, norm_w.data_ptr(), ctypes.c_float(EPS),
                                        ctypes.byref(p), _lib.logit_threshold(thr_p), lut.data_ptr(),
                                        slots.data_ptr(), ids.data_ptr(), counts.data_ptr(),
                                        dslots.data_ptr(), dids.data_ptr(), total.data_ptr(),
                                        ws.data_ptr(), wsb, None))
        torch.cuda.synchronize()
        xn = rmsnorm(xq, norm_w, EPS).double().cpu().numpy()   # the kernels' own normalisation
        q = query_for(xn, dtype)
        ref = O.predictor_logits(q, D, U, b)
        amb = O.ambiguous(ref, thr_p)
        want = O.cold_ids_for(ref >= O.logit_threshold(thr_p), hot_ids.cpu().tolist(), inter)
        got = chunked_ids(counts, ids)
        assert got == sorted(got)
        gs, ws_ = set(got), set(want)
        diff = gs ^ ws_
        assert all(amb[i] for i in diff), f"{len(diff)} ids differ outside the 1e-6 band"
        n = int(total.item())
        assert n == len(got)
        assert dids[:n].cpu().tolist() == got
        assert dslots[:n].cpu().tolist() == [3 * i for i in got]


def test_batch_query_equals_mean_of_the_normalisation(dev):
    """engine.py:277 at batch 8 on many batches: the device's query (the
    fp16 batch mean of RMSNorm(x), cast to bf16, left in the predictor
    workspace) equals the oracle's mean over oi2_rmsnorm's rows bit for bit,
    so the selection equals the oracle's outside the 1e-6 band.  The norm
    arithmetic must round every kernel's product the same way: a fused
    multiply-and-round in one kernel and not in another gave one-ulp
    differences in about one layer in seven."""
    import ctypes
    g = torch.Generator(device=dev).manual_seed(77)
    inter = 14336
    pred = random_predictor(g, inter, 64, torch.bfloat16, dev)
    D, U, b = pred_weights(pred)
    norm_w = (1 + 0.05 * torch.randn(H, generator=g, device=dev)).half()
    lut = torch.arange(inter, dtype=torch.int32, device=dev)
    nc = (inter + 255) // 256
    slots = torch.empty(nc * 256, dtype=torch.int32, device=dev)
    ids = torch.empty_like(slots)
    counts = torch.empty(nc, dtype=torch.int32, device=dev)
    p = pred.struct()
    L = _lib.lib()
    wsb = L.oi2_predict_workspace_bytes(ctypes.byref(p))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    for k in range(24):
        xq = (torch.randn((8, H), generator=g, device=dev) * (0.5 + k / 8)).half()
        _lib.check(L.oi2_predict_select(xq.data_ptr(), 8, norm_w.data_ptr(), ctypes.c_float(EPS),
                                        ctypes.byref(p), 0.0, lut.data_ptr(), slots.data_ptr(),
                                        ids.data_ptr(), counts.data_ptr(), None, None, None,
                                        ws.data_ptr(), wsb, None))
        torch.cuda.synchronize()
        q_dev = ws[:4 * H].view(torch.float32).double().cpu().numpy()
        q = query_for(rmsnorm(xq, norm_w, EPS).double().cpu().numpy(), torch.bfloat16)
        assert np.array_equal(q_dev, q), f"batch {k}: {int((q_dev != q).sum())} query elements differ"
        ref = O.predictor_logits(q, D, U, b)
        want = O.cold_ids_for(ref >= 0.0, [], inter)
        got = chunked_ids(counts, ids)
        amb = O.ambiguous(ref, 0.5)
        assert all(amb[i] for i in set(got) ^ set(want)), f"batch {k}: ids differ outside the band"


def test_predictor_registry_predict_from_files(dev):
    """PredictorRegistry.predict exactly as _cold_ids_for calls it
    (engine.py:277-278): an fp32 predictor file (as predictor.py saves it),
    hidden states of each float dtype cast straight to fp32, masks equal to
    the oracle outside the band; a layer without a file gives None; and the
    p == 1 edge selects exactly the logits whose float32 sigmoid is 1.0."""
    g = torch.Generator(device=dev).manual_seed(57)
    inter = 4096
    pred = random_predictor(g, inter, 64, torch.float32, dev)
    # neurons 0..3 have zero up rows, so their logit is their bias alone,
    # placed on either side of the float32 sigmoid's saturation point
    z1 = np.float32(O.sigmoid_f32_threshold(1.0))
    edge = [np.nextafter(z1, np.float32(0)), z1, np.nextafter(z1, np.float32(99)), np.float32(17)]
    pred.up_w[:4] = 0.0
    pred.up_b[:4] = torch.tensor(edge, dtype=torch.float32, device=dev)
    with tempfile.TemporaryDirectory() as tmp:
        pred.save(os.path.join(tmp, "layer_005_expert_000.pt"))
        reg = oi2.PredictorRegistry(tmp, device=dev)
        assert reg.predict(4, 0, torch.zeros(H, device=dev)) is None
        D, U, b = pred_weights(pred)
        for h_dtype in (torch.float16, torch.float32, torch.bfloat16):
            h = (torch.randn((1, H), generator=g, device=dev) * 0.8).to(h_dtype)
            for thr in (0.5, 0.6, 1.0):
                mask = reg.predict(5, 0, h, thr)
                assert mask.shape == (1, inter) and mask.dtype == torch.bool
                ref = O.predictor_logits(h.float().cpu().numpy().astype(np.float64), D, U, b)[0]
                want = ref >= O.logit_threshold(thr)
                amb = O.ambiguous(ref, thr)
                got = mask[0].cpu().numpy()
                assert np.array_equal(got[~amb], want[~amb]), (h_dtype, thr)
                if thr == 1.0:
                    sig = torch.sigmoid(torch.tensor(edge, dtype=torch.float32))
                    assert got[:4].tolist() == (sig >= 1.0).tolist() == [False, True, True, True]
                    assert not got[4:].any()


# ── sparse_ffn on the reference's own tensors ───────────────────────────────

@pytest.fixture(scope="module")
def config1_files(dev):
    """Survey config 1's layer written as split files: 2867 hot neurons in a
    reference-layout hot .pt (fp8, no scales) and the other 11469 as INT4
    records in a cold file, plus the dense weights."""
    g = torch.Generator(device=dev).manual_seed(61)
    inter = 14336
    lay = SyntheticLayer(g, inter, 2867, device=dev, keep_dense=True, per_row_scale=False)
    tmp = tempfile.TemporaryDirectory()
    w = oi2.format.ColdFileWriter(os.path.join(tmp.name, "cold_weights.bin"), 1)
    w.add_section(0, lay.records.cpu().numpy())
    w.close(os.path.join(tmp.name, "cold_index.npy"))
    cfg = {"hidden_dim": H, "intermediate_dim": inter, "rms_norm_eps": EPS, "num_experts": 1}
    store = oi2.ColdWeightStore(os.path.join(tmp.name, "cold_weights.bin"),
                                os.path.join(tmp.name, "cold_index.npy"), cfg, device=dev)
    gate, up, down = lay.dense
    hid = lay.hot_ids
    fp8 = {"gate": gate[hid].to(torch.float8_e4m3fn), "up": up[hid].to(torch.float8_e4m3fn),
           "down": down[:, hid].to(torch.float8_e4m3fn)}
    yield lay, g, store, fp8
    store.close()
    tmp.cleanup()


@pytest.mark.parametrize("B,activation,both", [(1, "silu", False), (5, "silu", False),
                                               (3, "relu", True)])
def test_sparse_ffn_takes_the_reference_call(dev, config1_files, B, activation, both):
    """sparse_ffn exactly as engine.py:302-307 calls it: hot gate/up/down as
    SparseFFNLayer widens them from the hot file (fp16, engine.py:255-261),
    cold gate/up/down as read_neurons returns them (fp32, (N,H)/(N,H)/(H,N)),
    for 10 % of the cold neurons (config 1).  Against the float64 oracle over
    the same tensors, and against the fused fp8/INT4 path on the same
    weights; n_hot 2867 leaves the down rows unaligned."""
    lay, g, store, fp8 = config1_files
    gh, uh, dh = (fp8[k].to(torch.float16) for k in ("gate", "up", "down"))
    cold_ids = lay.cold_ids[torch.randperm(lay.cold_ids.numel(), generator=g, device=dev)[:1147]]
    ids = cold_ids.cpu().tolist()
    gc, uc, dc = store.read_neurons(0, 0, ids)
    assert gc.dtype == torch.float32 and dc.shape == (H, 1147)
    x = rmsnorm(torch.randn((B, H), generator=g, device=dev).half(), lay.norm_w, EPS)
    y = oi2.sparse_ffn(x, activation, both, gh, uh, dh, gc, uc, dc)
    torch.cuda.synchronize()
    assert y.dtype == torch.float16 and y.shape == (B, H)
    f64 = lambda t: t.double().cpu().numpy()
    ref = O.sparse_ffn(f64(x), activation, both, f64(gh), f64(uh), f64(dh), f64(gc), f64(uc), f64(dc))
    for r in range(B):
        assert_ffn_close(f64(y[r]), ref[r], what=f"dense sparse_ffn row {r}")
    # the same weights through the fused kernels (fp8 codes, INT4 records)
    hot = oi2.HotWeights(lay.hot_ids, fp8["gate"].view(torch.uint8), fp8["up"].view(torch.uint8),
                         fp8["down"].view(torch.uint8), torch.ones(2867, device=dev),
                         torch.ones(2867, device=dev), torch.ones(H, device=dev))
    cold = ColdNeurons.from_ids(store.section(0), ids)
    y_fused = oi2.sparse_ffn(x, activation, both, hot, None, None, cold)
    assert_ffn_close(f64(y_fused), f64(y), tol=2e-3, cos_min=0.99999, what="fused vs dense")
    # one half as tensors, the other as a handle
    y_mixed = oi2.sparse_ffn(x, activation, both, gh, uh, dh, cold)
    assert_ffn_close(f64(y_mixed), f64(y), tol=2e-3, cos_min=0.99999, what="mixed")


def test_sparse_ffn_reference_call_edges(dev, config1_files):
    """Either half missing or empty (engine.py:194, :199), both empty giving
    zeros (:207-208), cold records read out of request order with duplicates,
    bf16 weights, fp32 and bf16 activations, and integer activations refused."""
    lay, g, store, fp8 = config1_files
    gh, uh, dh = (fp8[k].to(torch.float16) for k in ("gate", "up", "down"))
    ids = [int(lay.cold_ids[k]) for k in (40, 3, 3, 700, 11000, 5)]
    gc, uc, dc = store.read_neurons(0, 0, ids)
    x = rmsnorm(torch.randn((2, H), generator=g, device=dev).half(), lay.norm_w, EPS)
    f64 = lambda t: t.double().cpu().numpy()
    empty = torch.zeros((0, H), dtype=torch.float16, device=dev)
    cases = [((gh, uh, dh), (None, None, None), "hot only"),
             ((empty, empty, empty.t()), (gc, uc, dc), "cold only (empty hot tensors)"),
             ((None, None, None), (gc, uc, dc), "cold only"),
             ((gh.bfloat16(), uh.bfloat16(), dh.bfloat16()), (gc, uc, dc), "bf16 hot")]
    for hot, cold, what in cases:
        y = oi2.sparse_ffn(x, "silu", False, *hot, *cold)
        torch.cuda.synchronize()
        ref = O.sparse_ffn(f64(x), "silu", False, *(None if t is None else f64(t) for t in hot),
                           *(None if t is None else f64(t) for t in cold))
        for r in range(2):
            assert_ffn_close(f64(y[r]), ref[r], what=f"{what} row {r}")
    z = oi2.sparse_ffn(x, "silu", False, None, None, None, None, None, None)
    assert z.dtype == torch.float16 and torch.count_nonzero(z) == 0
    # activations of another float dtype, as engine.py:173-209 takes them:
    # the result comes back in x's dtype, against the oracle over x itself
    for xt in (x.float() * 1.0001, x.bfloat16()):
        y = oi2.sparse_ffn(xt, "silu", False, gh, uh, dh, gc, uc, dc)
        torch.cuda.synchronize()
        assert y.dtype == xt.dtype and y.shape == xt.shape
        ref = O.sparse_ffn(f64(xt), "silu", False, f64(gh), f64(uh), f64(dh), f64(gc), f64(uc), f64(dc))
        for r in range(2):
            assert_ffn_close(f64(y[r]), ref[r], what=f"{xt.dtype} activations row {r}")
    with pytest.raises(TypeError, match="floating point"):
        oi2.sparse_ffn(x.int(), "silu", False, gh, uh, dh, None, None, None)
    with pytest.raises(ValueError, match="gate/up must be"):
        oi2.sparse_ffn(x, "silu", False, gh, uh, dh.t(), None, None, None)


# ── drop-in layer from split files ───────────────────────────────────────────

def test_sparse_ffn_layer_from_split_files(dev):
    """SparseFFNLayer built exactly as DesdemonaEngine builds it
    (engine.py:391-398) from a hot .pt in the reference layout (fp8, no
    scales), a cold file and an fp32 predictor file."""
    g = torch.Generator(device=dev).manual_seed(41)
    inter = 14336
    lay = SyntheticLayer(g, inter, 3584, device=dev, keep_dense=True, per_row_scale=False,
                         std=0.05)
    gate, up, down = lay.dense
    with tempfile.TemporaryDirectory() as tmp:
        hot_dir = os.path.join(tmp, "hot_weights")
        os.makedirs(hot_dir)
        hid = lay.hot_ids
        torch.save({"neuron_ids": hid.cpu(), "gate": gate[hid].cpu().to(torch.float8_e4m3fn),
                    "up": up[hid].cpu().to(torch.float8_e4m3fn),
                    "down": down[:, hid].cpu().to(torch.float8_e4m3fn)},
                   os.path.join(hot_dir, "layer_002_expert_000.pt"))
        w = oi2.format.ColdFileWriter(os.path.join(tmp, "cold_weights.bin"), 3)
        empty = np.zeros((0, 6400), np.uint8)
        w.add_section(0, empty)
        w.add_section(1, empty)
        w.add_section(2, lay.records.cpu().numpy())
        w.close(os.path.join(tmp, "cold_index.npy"))
        pdir = os.path.join(tmp, "pred")
        os.makedirs(pdir)
        pred = random_predictor(g, inter, 64, torch.float32, dev)
        pred.save(os.path.join(pdir, "layer_002_expert_000.pt"))
        cfg = {"hidden_dim": H, "intermediate_dim": inter, "hidden_act": "silu",
               "act_on_both": False, "rms_norm_eps": EPS, "num_experts": 1}
        store = oi2.ColdWeightStore(os.path.join(tmp, "cold_weights.bin"),
                                    os.path.join(tmp, "cold_index.npy"), cfg, device=dev)
        reg = oi2.PredictorRegistry(pdir, device=dev)
        layer = oi2.SparseFFNLayer(2, hot_dir, store, reg, cfg, dev, None,
                                   ffn_norm_weight=lay.norm_w.cpu())
        x = torch.randn((1, 1, H), generator=g, device=dev).half()
        y_direct = layer(x)
        fut = layer.submit_cold_fetch(x)
        y_pref = layer(x, fut)
        torch.cuda.synchronize()
        assert torch.equal(y_direct, y_pref)
        xn_gpu = rmsnorm(x, lay.norm_w, EPS)
        ids = layer._cold_ids_for(xn_gpu)
        xn = normed_f16(x[0], lay.norm_w)
        D, U, b = pred_weights(pred)
        ref_logits = O.predictor_logits(xn_gpu[0, 0].double().cpu().numpy(), D, U, b)
        want = O.cold_ids_for(ref_logits >= 0.0, hid.cpu().tolist(), inter)
        diff = set(ids) ^ set(want)
        assert all(O.ambiguous(ref_logits)[i] for i in diff)
        sec = store.section(2)
        slots = sec.slots_for(ids)
        Gh = O.FP8_TABLE[gate[hid].cpu().to(torch.float8_e4m3fn).view(torch.uint8).numpy()]
        Uh = O.FP8_TABLE[up[hid].cpu().to(torch.float8_e4m3fn).view(torch.uint8).numpy()]
        Dh = O.FP8_TABLE[down[:, hid].cpu().to(torch.float8_e4m3fn).view(torch.uint8).numpy()]
        Gc, Uc, Dc = cold_dense(lay.records, slots)
        ref = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
        res = y_direct[0].float().cpu().numpy() - x[0].float().cpu().numpy()
        assert_ffn_close(res, ref, tol=1e-2, cos_min=0.9999, what="layer forward")
        # a layer with no predictor fetches every cold neuron (engine.py:282-283)
        layer_np = oi2.SparseFFNLayer(2, hot_dir, store, None, cfg, dev, None,
                                      ffn_norm_weight=lay.norm_w.cpu())
        y_all = layer_np(x)
        Gc, Uc, Dc = cold_dense(lay.records, np.arange(lay.records.shape[0]))
        ref_all = O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc)
        assert_ffn_close(y_all[0].float().cpu().numpy() - x[0].float().cpu().numpy(), ref_all,
                         what="no predictor")
        # layers with an empty cold section compute the hot half only
        store.close()


@pytest.mark.parametrize("direct_io", [False, True], ids=["mmap", "direct"])
def test_sparse_ffn_layer_file_residency(dev, direct_io):
    """The reference's memory model: ColdWeightStore(residency="file") keeps
    the records in the split file, and SparseFFNLayer fetches each layer's
    predicted records on the caller's executor (engine.py:266-290: read,
    then copy to the device), from the mapping or with O_DIRECT page reads.
    read_neurons equals the HBM-resident store's bit for bit; the layer's
    output equals the HBM-resident layer's to rounding and the oracle's within
    the FFN bar; a prefetched future and a direct forward agree exactly."""
    from concurrent.futures import ThreadPoolExecutor
    g = torch.Generator(device=dev).manual_seed(43)
    inter = 14336
    lay = SyntheticLayer(g, inter, 3584, device=dev, with_predictor=True, pred_dtype=torch.float32)
    with tempfile.TemporaryDirectory(dir=os.path.dirname(os.path.abspath(__file__))) as tmp:
        hot_dir = os.path.join(tmp, "hot")
        os.makedirs(hot_dir)
        lay.hot.save(os.path.join(hot_dir, "layer_000_expert_000.pt"))
        w = oi2.format.ColdFileWriter(os.path.join(tmp, "cold_weights.bin"), 1)
        w.add_section(0, lay.records.cpu().numpy())
        w.close(os.path.join(tmp, "cold_index.npy"))
        pdir = os.path.join(tmp, "pred")
        os.makedirs(pdir)
        lay.predictor.save(os.path.join(pdir, "layer_000_expert_000.pt"))
        cfg = {"hidden_dim": H, "intermediate_dim": inter, "hidden_act": "silu",
               "act_on_both": False, "rms_norm_eps": EPS, "num_experts": 1}
        paths = (os.path.join(tmp, "cold_weights.bin"), os.path.join(tmp, "cold_index.npy"))
        try:
            fstore = oi2.ColdWeightStore(*paths, cfg, device=dev, residency="file", direct_io=direct_io)
        except oi2.OI2Error as e:
            if direct_io and "O_DIRECT" in str(e):
                pytest.skip(f"this file system refuses O_DIRECT: {e}")
            raise
        hstore = oi2.ColdWeightStore(*paths, cfg, device=dev)
        reg = oi2.PredictorRegistry(pdir, device=dev)
        ex = ThreadPoolExecutor(max_workers=2)
        try:
            ids = [int(i) for i in lay.cold_ids[torch.randperm(lay.cold_ids.numel(), generator=g,
                                                               device=dev)[:300]].tolist()]
            ids += [ids[5], 10 ** 6]                      # a duplicate and an absent id
            a = fstore.read_neurons(0, 0, ids)
            b = hstore.read_neurons(0, 0, ids)
            torch.cuda.synchronize()
            assert all(torch.equal(u, v) for u, v in zip(a, b))
            lf = oi2.SparseFFNLayer(0, hot_dir, fstore, reg, cfg, dev, ex, ffn_norm_weight=lay.norm_w.cpu())
            lh = oi2.SparseFFNLayer(0, hot_dir, hstore, reg, cfg, dev, ex, ffn_norm_weight=lay.norm_w.cpu())
            # one token: the single-token kernels sum in a fixed order, so a
            # prefetched and a direct forward agree bit for bit
            x1 = torch.randn((1, 1, H), generator=g, device=dev).half()
            fut = lf.submit_cold_fetch(x1)
            y1_pref = lf(x1, fut)
            y1_dir = lf(x1)
            torch.cuda.synchronize()
            assert torch.equal(y1_pref, y1_dir)
            # two tokens (the batch kernels, whose split sums round in any order)
            x = torch.randn((2, 1, H), generator=g, device=dev).half()
            fut = lf.submit_cold_fetch(x)
            y_pref = lf(x, fut)
            y_dir = lf(x)
            y_hbm = lh(x)
            torch.cuda.synchronize()
            assert_ffn_close(y_pref.double().cpu().numpy().ravel(), y_dir.double().cpu().numpy().ravel(),
                             tol=1e-3, cos_min=0.999999, what="prefetched vs direct")
            assert_ffn_close(y_dir.double().cpu().numpy().ravel(), y_hbm.double().cpu().numpy().ravel(),
                             tol=2e-3, cos_min=0.99999, what="file vs HBM residency")
            # against the oracle: the layer's own selection, teacher-forced
            slots = lf._cold_slots_host(x, normed=False)
            xn = normed_f16(x[:, 0], lay.norm_w)
            ref = O.sparse_ffn(xn, "silu", False, *hot_dense(lay.hot), *cold_dense(lay.records, slots))
            res = y_dir[:, 0].double().cpu().numpy() - x[:, 0].double().cpu().numpy()
            for r in range(2):
                assert_ffn_close(res[r], ref[r], tol=1e-2, cos_min=0.9999, what=f"file residency row {r}")
        finally:
            ex.shutdown()
            fstore.close()
            hstore.close()
