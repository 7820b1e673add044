"""Pins the CPU oracle (and the library's host-side record writer) against the
reference's golden vectors, closed forms and brute force.  CPU only."""
import hashlib
import json
import os
import struct
import tempfile

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from oi2 import format as fmt
from tests.fixtures import synthetic_cold_file

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _golden(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


# ── golden byte image of the reference fixture writer ───────────────────────

@pytest.fixture(scope="module")
def seed0_file():
    with tempfile.TemporaryDirectory() as tmp:
        cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp, 4, 16, 0)
        raw = open(cold_bin, "rb").read()
        index = np.load(cold_idx)
        yield raw, index, layers


def test_writer_byte_image_matches_reference(seed0_file):
    raw, index, _ = seed0_file
    g = _golden("cold_seed0.json")
    assert len(raw) == g["file_bytes"]
    assert index.reshape(-1).tolist() == g["cold_index"]
    assert hashlib.sha256(raw).hexdigest() == g["file_sha256"]
    recs = np.load(os.path.join(GOLDEN, "cold_seed0_records.npy"))
    for li in range(4):
        off = int(index[li, 0, 0])
        for k in range(2):
            s = off + 16 + k * fmt.NEURON_RECORD_BYTES
            assert np.array_equal(np.frombuffer(raw[s:s + fmt.NEURON_RECORD_BYTES], np.uint8),
                                  recs[li * 2 + k])


def test_oracle_dequant_matches_reference_truth(seed0_file):
    """Every record of the golden file, decoded by the oracle, hashes to the
    reference's own dequantize_int4 output (tests/common.py:74-81)."""
    raw, index, _ = seed0_file
    g = _golden("cold_seed0.json")
    n_checked = 0
    for li in range(4):
        m = O.section_map(raw, index, li, 0)
        assert sorted(m) == sorted(g["nid_order"][str(li)])
        for nid, off in m.items():
            _, ga, up, dn = O.record_vectors(raw, off)
            for name, v in (("gate", ga), ("up", up), ("down", dn)):
                h = hashlib.sha256(v.astype("<f4").tobytes()).hexdigest()
                assert h == g["truth_sha256"][f"{li}:{nid}:{name}"], (li, nid, name)
                n_checked += 1
    assert n_checked == 4 * 16 * 3


def test_quantize_edge_cases_match_reference():
    q = _golden("quant_edge.json")
    for name, case in q.items():
        x = np.frombuffer(bytes.fromhex(case["x_f32_hex"]), dtype="<f4")
        packed_o, scales_o = O.quantize_int4_ref(x)
        packed_l, scales_l = fmt.quantize_int4(x)
        assert packed_o.hex() == case["packed_hex"], name
        assert packed_l.hex() == case["packed_hex"], name
        assert scales_o.astype("<f4").tobytes().hex() == case["scales_f32_hex"], name
        assert scales_l.astype("<f4").tobytes().hex() == case["scales_f32_hex"], name
        assert scales_l.astype(np.float16).tobytes().hex() == case["scales_f16_hex"], name


# ── dequant closed form ──────────────────────────────────────────────────────

def test_dequant_exhaustive_bytes():
    """Every byte value in every position of a group, against the two's
    complement definition computed independently of the oracle."""
    packed = np.arange(256, dtype=np.uint8)
    packed = np.tile(packed, 16)               # 4096 bytes -> 8192 elements
    scales = np.array([0.5, -1.25, 3.0, 1e-3] * 16, dtype=np.float32)
    out = O.dequant_int4(packed, scales, 8192)
    for i in range(8192):
        byte = int(packed[i // 2])
        nib = (byte >> 4) if i % 2 else (byte & 15)
        signed = nib - 16 if nib >= 8 else nib
        assert out[i] == np.float32(signed) * scales[i // 128]
    # the product nibble * fp16-valued scale is exact in fp32
    s16 = np.float16(0.0173).astype(np.float32)
    vals = O.dequant_int4(np.array([0x8F, 0x7E], np.uint8), np.array([s16]), 4)
    assert np.array_equal(vals.astype(np.float64), np.array([-1, -8, -2, 7]) * np.float64(s16))


def test_quant_invariants():
    """tests/test_quantization.py:17-63 restated on the oracle quantiser."""
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(4096, generator=g) * 3.0).numpy()
    p, s = O.quantize_int4_ref(x)
    y = O.dequant_int4(p, s, 4096)
    err = np.abs(y - x).reshape(-1, 128).max(1)
    bound = np.maximum(np.abs(x.reshape(-1, 128)).max(1), 1e-8) / 7.0 / 2.0
    assert (err <= bound + 1e-6).all()
    p, s = O.quantize_int4_ref(np.zeros(4096, np.float32))
    assert np.all(O.dequant_int4(p, s, 4096) == 0)
    assert len(O.quantize_int4_ref(x)[0]) == 2048
    x100 = (torch.randn(100, generator=g)).numpy()
    p, s = O.quantize_int4_ref(x100)
    assert np.abs(O.dequant_int4(p, s, 100) - x100).max() <= np.abs(x100).max() / 14 + 1e-6
    xe = np.array([100.0, -100.0, 50.0, -50.0] * 32, np.float32)
    p, s = O.quantize_int4_ref(xe)
    ye = O.dequant_int4(p, s, 128)
    assert np.all(np.sign(ye) == np.sign(xe))


# ── record access semantics (tests/test_cold_store.py:28-91) ────────────────

def test_read_neurons_semantics(seed0_file):
    raw, index, layers = seed0_file
    nids, G, U, D = layers[0]
    # exact values with fp16-rounded scales, shapes (1,H)/(H,1)
    out = O.read_neurons(raw, index, 0, 0, [nids[3]])
    assert out[0].shape == (1, 4096) and out[2].shape == (4096, 1)
    p, s = fmt.quantize_int4(G[3])
    assert np.array_equal(out[0][0], O.dequant_int4(p, s.astype(np.float16).astype(np.float32), 4096))
    # request order, duplicates kept, absent skipped
    req = [nids[5], 10_000, nids[1], nids[5]]
    g, u, d = O.read_neurons(raw, index, 0, 0, req)
    assert g.shape == (3, 4096) and d.shape == (4096, 3)
    assert np.array_equal(g[0], g[2])
    assert not np.array_equal(g[0], g[1])
    assert O.read_neurons(raw, index, 0, 0, [10_000, 10_001]) is None
    empty_index = index.copy()
    empty_index[1, 0, 1] = 0
    assert O.read_neurons(raw, empty_index, 1, 0, [layers[1][0][0]]) is None


# ── FP8 decode ───────────────────────────────────────────────────────────────

def test_fp8_table_matches_torch_and_spec():
    codes = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn)
    t = codes.to(torch.float32).numpy().astype(np.float64)
    nan = np.isnan(O.FP8_TABLE)
    assert np.array_equal(np.isnan(t), nan)
    assert nan.sum() == 2
    assert np.array_equal(t[~nan], O.FP8_TABLE[~nan])
    assert O.FP8_TABLE[0x7E] == 448.0 and O.FP8_TABLE[0x01] == 2.0 ** -9
    assert O.FP8_TABLE[0x38] == 1.0 and O.FP8_TABLE[0xB8] == -1.0


# ── FFN math ────────────────────────────────────────────────────────────────

def _brute_ffn(x, G, U, D, act, both):
    n, H = G.shape
    y = [0.0] * D.shape[0]
    for k in range(n):
        g = sum(G[k][i] * x[i] for i in range(H))
        u = sum(U[k][i] * x[i] for i in range(H))
        if act == "relu":
            a = max(g, 0.0) * (max(u, 0.0) if both else u)
        else:
            sg = g / (1.0 + np.exp(-g))
            a = sg * ((u / (1.0 + np.exp(-u))) if both else u)
        for j in range(D.shape[0]):
            y[j] += D[j][k] * a
    return np.array(y)


@pytest.mark.parametrize("act,both", [("silu", False), ("relu", True), ("relu", False), ("gelu", False)])
def test_sparse_ffn_brute_force_and_torch(act, both):
    rng = np.random.default_rng(3)
    H, nh, nc = 12, 5, 3
    x = rng.standard_normal(H)
    Gh, Uh = rng.standard_normal((nh, H)), rng.standard_normal((nh, H))
    Dh = rng.standard_normal((H, nh))
    Gc, Uc = rng.standard_normal((nc, H)), rng.standard_normal((nc, H))
    Dc = rng.standard_normal((H, nc))
    y = O.sparse_ffn(x, act, both, Gh, Uh, Dh, Gc, Uc, Dc)
    eff = "relu" if act == "relu" else "silu"
    yb = _brute_ffn(x, Gh, Uh, Dh, eff, both) + _brute_ffn(x, Gc, Uc, Dc, eff, both)
    np.testing.assert_allclose(y, yb, rtol=1e-12, atol=1e-12)
    # engine.py:194-205 written with torch's own linear/activations
    tx = torch.from_numpy(x)[None]
    fn = F.relu if act == "relu" else F.silu

    def half(G, U, D):
        g, u = F.linear(tx, torch.from_numpy(G)), F.linear(tx, torch.from_numpy(U))
        return F.linear(fn(g) * (fn(u) if both else u), torch.from_numpy(D))
    yt = (half(Gh, Uh, Dh) + half(Gc, Uc, Dc))[0].numpy()
    np.testing.assert_allclose(y, yt, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("both", [False, True])
def test_decomposition_exact(both):
    """tests/test_ffn_exactness.py:51-79 at real H with quantised halves."""
    rng = np.random.default_rng(11)
    H, n = 4096, 48
    x = rng.standard_normal(H)
    G = rng.standard_normal((n, H)) * 0.05
    U = rng.standard_normal((n, H)) * 0.05
    D = rng.standard_normal((H, n)) * 0.05
    act = "relu" if both else "silu"
    full = O.sparse_ffn(x, act, both, G, U, D, None, None, None)
    split = O.sparse_ffn(x, act, both, G[:20], U[:20], D[:, :20], G[20:], U[20:], D[:, 20:])
    np.testing.assert_allclose(full, split, rtol=1e-10, atol=1e-12)
    assert np.all(O.sparse_ffn(x, act, both, None, None, None, None, None, None) == 0)
    # linear in the down weights, zero when every gate is negative under relu
    np.testing.assert_allclose(O.sparse_ffn(x, act, both, G, U, 2 * D, None, None, None), 2 * full)
    Gneg = -np.abs(G) * np.sign(x)[None, :]
    y0 = O.sparse_ffn(np.abs(x) * np.sign(x), "relu", both, Gneg, U, D, None, None, None)
    assert np.all(y0 == 0)


def test_silu_closed_form():
    assert O.silu(0.0) == 0.0
    assert abs(O.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-15
    assert abs(O.silu(40.0) - 40.0) < 1e-12 and abs(O.silu(-40.0)) < 1e-15


def test_rmsnorm_matches_torch():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((3, 4096))
    w = rng.standard_normal(4096)
    m = torch.nn.RMSNorm(4096, eps=1e-5).double()
    m.weight.data = torch.from_numpy(w)
    ref = m(torch.from_numpy(x)).detach().numpy()
    np.testing.assert_allclose(O.rmsnorm(x, w, 1e-5), ref, rtol=1e-12, atol=1e-12)


# ── predictor ────────────────────────────────────────────────────────────────

def test_predictor_mask_matches_sigmoid_threshold():
    """tests/test_predictor.py:78-85 restated: mask == (probs >= thr), with
    probs from torch Linear layers in float64."""
    torch.manual_seed(0)
    H, I, R = 256, 128, 32
    down = torch.nn.Linear(H, R, bias=False).double()
    up = torch.nn.Linear(R, I, bias=True).double()
    x = torch.randn(4, H, dtype=torch.float64)
    probs = torch.sigmoid(up(down(x))).detach().numpy()
    logits = O.predictor_logits(x.numpy(), down.weight.detach().numpy(),
                                up.weight.detach().numpy(), up.bias.detach().numpy())
    np.testing.assert_allclose(1 / (1 + np.exp(-logits)), probs, rtol=1e-12)
    for thr in (0.5, 0.3, 0.77):
        m = O.predict_mask(x.numpy(), down.weight.detach().numpy(),
                           up.weight.detach().numpy(), up.bias.detach().numpy(), thr)
        amb = O.ambiguous(logits, thr)
        assert np.array_equal(m[~amb], (probs >= thr)[~amb])


def test_cold_ids_for_order_and_hot_filter():
    mask = np.zeros(20, bool)
    mask[[17, 2, 5, 9, 11]] = True
    assert O.cold_ids_for(mask, [5, 11, 13], 20) == [2, 9, 17]
    assert O.cold_ids_for(None, [0, 1, 2], 6) == [3, 4, 5]


# ── casts and the batch query (predictor.py:455, engine.py:277) ─────────────

def test_to_bf16_matches_torch_cast():
    """oracle.to_bf16 against torch's own float32 -> bfloat16 cast, bit for
    bit: round-half-even ties both ways, +-0, subnormals, the largest finite
    values (which round to inf), infinities, and NaN (NaN either way)."""
    rng = np.random.default_rng(11)
    bits = [0x00000000, 0x80000000, 0x00000001, 0x807FFFFF, 0x00400000, 0x00008000, 0x00018000,
            0x3F808000, 0x3F818000, 0x3F807FFF, 0x3F808001, 0xBF808000, 0xBF818000,
            0x7F7FFFFF, 0xFF7FFFFF, 0x7F7F7FFF, 0x7F7F8000, 0x7F800000, 0xFF800000,
            0x7FC00000, 0xFFC00000, 0x7F800001, 0x7FBFFFFF]
    # ties: the low 16 bits exactly 0x8000, both parities of bit 16
    ties = (rng.integers(0, 1 << 15, 20000, dtype=np.uint64) << 17) | 0x8000
    ties |= rng.integers(0, 2, 20000, dtype=np.uint64) << 16
    rand = rng.integers(0, 1 << 32, 200000, dtype=np.uint64)
    f = np.concatenate([np.array(bits, np.uint64), ties, rand]).astype(np.uint32).view(np.float32)
    got = O.to_bf16(f)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # the same through the usual path of the predictor query: fp16 values
    h = rng.standard_normal(100000).astype(np.float16).astype(np.float32)
    assert np.array_equal(O.to_bf16(h).view(np.uint32),
                          torch.from_numpy(h).to(torch.bfloat16).float().numpy().view(np.uint32))


@pytest.mark.parametrize("rows", [1, 3, 8])
def test_query_matches_torch_fp16_batch_mean(rows):
    """oracle.query is engine.py:277's ``x_normed[:, -1, :].mean(0)`` over fp16
    rows: torch's fp16 mean, bit for bit, on normal rows and on rows of mixed
    scale (where fp32 accumulation order could matter)."""
    rng = np.random.default_rng(rows)
    for scale in (1.0, None):
        x = rng.standard_normal((rows, 100000))
        if scale is None:
            x *= 10.0 ** rng.integers(-4, 4, (rows, 1))
        x16 = x.astype(np.float16)
        want = torch.from_numpy(x16).mean(0).numpy()
        got = O.query(x16)
        assert got.dtype == np.float16
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # the engine's own shape: (B, T, H) normalised states, last position
    xt = torch.from_numpy(rng.standard_normal((rows, 3, 4096)).astype(np.float16))
    want = xt[:, -1, :].mean(0, keepdim=True).numpy()
    assert np.array_equal(O.query(xt[:, -1, :].numpy())[None].view(np.uint16),
                          want.view(np.uint16))


def test_threshold_edges_follow_float32_sigmoid():
    """The logit cut at the threshold's edges: p == 1 passes exactly the
    logits whose float32 sigmoid is 1.0, p > 1 none and p <= 0 all
    (predictor.py:77-79 in float32); away from the edges the cut is within
    the 1e-6 exemption band of torch's float32 decision."""
    z0 = O.sigmoid_f32_threshold(1.0)
    assert 16.6 < z0 < 16.7
    z = np.array([np.nextafter(z0, np.float32(0)), z0, np.nextafter(z0, np.float32(99)), 20.0,
                  -20.0, 0.0, 40.0], np.float32)
    sig = torch.sigmoid(torch.from_numpy(z))
    for p in (1.0, 1.5, 0.0, -0.5):
        want = (sig >= p).numpy()
        assert np.array_equal(z >= O.logit_threshold(p), want), p
    assert O.logit_threshold(1.0) == float(z0)
    rng = np.random.default_rng(4)
    for p in (0.5, 0.05, 0.637, 0.9):
        t = O.logit_threshold(p)
        zz = (t + rng.uniform(-1e-5, 1e-5, 20000)).astype(np.float32)
        want = (torch.sigmoid(torch.from_numpy(zz)) >= p).numpy()
        got = zz.astype(np.float64) >= t
        diff = got != want
        assert (np.abs(zz[diff].astype(np.float64) - t) <= 1e-6).all(), p
