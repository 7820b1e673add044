"""CPU oracle for the hot/cold sparse-FFN decode path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library imports this module;
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker.

Each function restates the reference's algorithm from its text (cited
file:line into the reference checkout) in numpy, computing in float64 where the
reference computes in floating point, so that the HIP path can be compared
against exact math over the same quantised weights.

Pins (see tests/test_oracle.py):
  dequant_int4      exhaustive 256-byte table x sign; golden truth hashes from
                    the reference fixture writer; exact-product argument
  read_neurons      golden file image: order, skip-absent, None, duplicates
  fp8 decode        OCP E4M3FN closed form; torch's own fp8->fp32 cast
  gated_act/ffn     hot+cold decomposition equals the one-pass FFN
                    (tests/test_ffn_exactness.py:79); brute-force tiny case;
                    relu sign cases; linearity in down weights; silu closed form
  rmsnorm           closed form against torch.nn.RMSNorm in float64
  predictor         predict_mask == sigmoid(logits) >= thr
                    (tests/test_predictor.py:78-85); logit-space threshold
                    equivalence; ascending order as nonzero()
  rope_cache        closed form: cos^2 + sin^2 = 1, position 0 is (1, 0),
                    angle t * theta^(-i/half) against torch's float32 table
  apply_rope        position 0 is the identity, pair norms are kept, the dot
                    of q at m and k at n depends on m - n only, rotating by p1
                    then p2 equals rotating by p1 + p2
  attention_core    torch's scaled_dot_product_attention (float64, with
                    enable_gqa) on random and causal cases; one key returns
                    its value; equal keys return the mean of the values
  gqa_attention     the composition above with torch.nn.RMSNorm and
                    F.linear in float64
"""
from __future__ import annotations

import math
import struct

import numpy as np

HIDDEN_DIM = 4096
GROUP = 128
VEC_BYTES = HIDDEN_DIM // 2
SCALE_BYTES_PER_VEC = (HIDDEN_DIM // GROUP) * 2
RECORD_BYTES = 6400
HEADER_BYTES = 16


# ── INT4 (splitter.py:81-124) ───────────────────────────────────────────────

def dequant_int4(packed, scales, N: int, group: int = GROUP) -> np.ndarray:
    """splitter.py:111-124: byte b -> (b & 0xF, b >> 4) interleaved low first,
    nibble > 7 -> nibble - 16, times float32(scale[i // group])."""
    arr = np.frombuffer(bytes(packed), dtype=np.uint8) if not isinstance(packed, np.ndarray) \
        else packed.astype(np.uint8).reshape(-1)
    lo = (arr & 0x0F).astype(np.int32)
    hi = ((arr >> 4) & 0x0F).astype(np.int32)
    flat = np.stack([lo, hi], axis=1).reshape(-1)[:N]
    flat = np.where(flat > 7, flat - 16, flat).astype(np.float32)
    scales = np.asarray(scales, dtype=np.float32).reshape(-1)
    n_groups = (N + group - 1) // group
    return flat * np.repeat(scales[:n_groups], group)[:N]


def quantize_int4_ref(x, group: int = GROUP):
    """splitter.py:81-108, one vector at a time as the reference does."""
    x = np.asarray(x, dtype=np.float32).reshape(-1)
    N = x.size
    if N % group:
        x = np.concatenate([x, np.zeros(group - N % group, np.float32)])
    g = x.reshape(-1, group)
    s = np.maximum(np.abs(g).max(axis=1), np.float32(1e-8)) / np.float32(7.0)
    q = np.clip(np.round(g / s[:, None]), -8, 7).astype(np.int8).reshape(-1)[:N]
    if N % 2:
        q = np.concatenate([q, np.zeros(1, np.int8)])
    lo = q[0::2].view(np.uint8) & 0x0F
    hi = (q[1::2].view(np.uint8) & 0x0F) << 4
    return (lo | hi).astype(np.uint8).tobytes(), s.astype(np.float32)


# ── record / section access (splitter.py:317-403) ─────────────────────────────

def record_vectors(buf, rec_off: int, H: int = HIDDEN_DIM):
    """Decode one record at byte offset ``rec_off``: returns (nid, gate, up, down)
    float32 vectors, as the loop body of splitter.py:370-395 does."""
    nid = struct.unpack_from("<H", buf, rec_off)[0]
    off = rec_off + 2
    vb = H // 2
    sb = (H // GROUP) * 2
    vecs = []
    for k in range(3):
        packed = bytes(buf[off + k * vb: off + (k + 1) * vb])
        s_off = off + 3 * vb + k * sb
        scales = np.frombuffer(bytes(buf[s_off:s_off + sb]), dtype=np.float16).astype(np.float32)
        vecs.append(dequant_int4(packed, scales, H))
    return nid, vecs[0], vecs[1], vecs[2]


def section_map(buf, index, layer: int, expert: int = 0, record_bytes: int = RECORD_BYTES):
    """splitter.py:332-352: nid -> byte offset of its record; None when the
    section is empty.  A duplicated id maps to its last record."""
    off, n = (int(v) for v in index[layer, expert])
    if n == 0:
        return None
    cur = off + HEADER_BYTES
    out = {}
    for _ in range(n):
        out[struct.unpack_from("<H", buf, cur)[0]] = cur
        cur += record_bytes
    return out


def read_neurons(buf, index, layer: int, expert: int, ids, H: int = HIDDEN_DIM):
    """splitter.py:354-403: request order, absent ids skipped, duplicates kept;
    returns (gate (N,H), up (N,H), down (H,N)) float32 or None."""
    m = section_map(buf, index, layer, expert)
    if m is None:
        return None
    g, u, d = [], [], []
    for nid in ids:
        if nid not in m:
            continue
        _, a, b, c = record_vectors(buf, m[nid], H)
        g.append(a)
        u.append(b)
        d.append(c)
    if not g:
        return None
    return np.stack(g), np.stack(u), np.stack(d, axis=1)


# ── FP8 e4m3fn (the hot weights' storage type, splitter.py:223-225) ─────────

def fp8_e4m3fn_decode(code: int) -> float:
    """OCP 8-bit floating point E4M3 (the FN variant): bias 7, no infinities,
    S.1111.111 is NaN, exponent 0 is subnormal (m/8 * 2^-6)."""
    s = -1.0 if code & 0x80 else 1.0
    e = (code >> 3) & 0xF
    m = code & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


FP8_TABLE = np.array([fp8_e4m3fn_decode(c) for c in range(256)], dtype=np.float64)


def fp8_dequant(codes, scales=None, axis: int = 1) -> np.ndarray:
    """fp8 codes -> float64 values times an optional per-row (axis 1) or
    per-column scale."""
    w = FP8_TABLE[np.asarray(codes, dtype=np.uint8)]
    if scales is not None:
        s = np.asarray(scales, dtype=np.float64)
        w = w * (s[:, None] if axis == 1 else s[None, :])
    return w


# ── FFN math (engine.py:163-209) ──────────────────────────────────────────────

def silu(v):
    v = np.asarray(v, dtype=np.float64)
    return v / (1.0 + np.exp(-v))


def gated_act(g, u, activation: str, act_on_both: bool):
    """engine.py:163-170: relu when activation == "relu", else silu (any other
    string falls back to silu); act(g)*act(u) when act_on_both, else act(g)*u."""
    act = (lambda v: np.maximum(v, 0.0)) if activation == "relu" else silu
    g = np.asarray(g, dtype=np.float64)
    u = np.asarray(u, dtype=np.float64)
    return act(g) * act(u) if act_on_both else act(g) * u


def sparse_ffn(x, activation, act_on_both, gate_hot, up_hot, down_hot,
               gate_cold, up_cold, down_cold, gate_bias_hot=None, gate_bias_cold=None):
    """engine.py:173-209 in float64: y = Dh act(Gh x, Uh x) + Dc act(Gc x, Uc x).
    Weights are dense (already dequantised); down matrices are (H, n).  An empty
    or missing half contributes nothing; both empty gives zeros (:207-208).
    ``gate_bias_*`` is the optional per-neuron gate pre-activation shift the
    sparse-firing workloads use (zero reproduces the reference)."""
    x = np.asarray(x, dtype=np.float64)
    squeeze = x.ndim == 1
    if squeeze:
        x = x[None, :]
    y = np.zeros_like(x)
    for G, U, D, b in ((gate_hot, up_hot, down_hot, gate_bias_hot),
                       (gate_cold, up_cold, down_cold, gate_bias_cold)):
        if G is None or np.asarray(G).shape[0] == 0:
            continue
        G = np.asarray(G, np.float64)
        U = np.asarray(U, np.float64)
        D = np.asarray(D, np.float64)
        g = x @ G.T
        if b is not None:
            g = g + np.asarray(b, np.float64)[None, :]
        h = gated_act(g, x @ U.T, activation, act_on_both)
        y = y + h @ D.T
    return y[0] if squeeze else y


def rmsnorm(x, weight, eps: float):
    """torch.nn.RMSNorm as used at engine.py:247-249 and :295:
    x / sqrt(mean(x^2) + eps) * weight, in float64."""
    x = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(weight, dtype=np.float64)


# ── predictor (predictor.py:55-79, 435-456; engine.py:274-283) ──────────────

def predictor_logits(h, D, U, b):
    """predictor.py:70-75 before the sigmoid: U (D h) + b, in float64 over the
    stored weights (predictor.py:67-68: down has no bias, up has one)."""
    h = np.asarray(h, dtype=np.float64)
    z = h @ np.asarray(D, np.float64).T
    return z @ np.asarray(U, np.float64).T + np.asarray(b, np.float64)


def logit_threshold(p: float) -> float:
    """sigmoid(l) >= p  <=>  l >= log(p / (1 - p)) for 0 < p < 1.  At the
    edges the reference's float32 sigmoid decides (predictor.py:75-79): every
    logit passes p <= 0; p == 1 passes the logits whose float32 sigmoid rounds
    to 1.0 (sigmoid_f32_threshold); p > 1 passes none."""
    if p <= 0.0:
        return -math.inf
    if p > 1.0:
        return math.inf
    if p == 1.0:
        return float(sigmoid_f32_threshold(1.0))
    return math.log(p / (1.0 - p))


def sigmoid_f32(z):
    """torch.sigmoid in float32 (predictor.py:75): 1 / (1 + exp(-z)), each
    step rounded to float32."""
    z = np.asarray(z, dtype=np.float32)
    one = np.float32(1.0)
    with np.errstate(over="ignore"):
        return one / (one + np.exp(-z, dtype=np.float32))


def _f32_key(v):
    """float32 -> an integer that orders like the float (ordered bit pattern)."""
    u = int(np.array(v, np.float32).view(np.uint32))
    return u ^ 0xFFFFFFFF if u >> 31 else u | 0x80000000


def _f32_from_key(k):
    u = k ^ 0xFFFFFFFF if not k >> 31 else k & 0x7FFFFFFF
    return np.array(u, np.uint32).view(np.float32)[()]


def sigmoid_f32_threshold(p: float) -> np.float32:
    """Smallest float32 logit z with sigmoid_f32(z) >= p (bisection over the
    ordered float32 bit patterns; sigmoid_f32 is non-decreasing), so that
    ``logit >= z`` is exactly the reference's float32 test
    ``sigmoid(logit) >= p`` (predictor.py:79).  +inf when no finite logit
    passes."""
    lo, hi = _f32_key(np.float32(-np.inf)), _f32_key(np.float32(np.inf))
    if sigmoid_f32(_f32_from_key(lo)) >= p:
        return np.float32(-np.inf)
    if not sigmoid_f32(_f32_from_key(hi - 1)) >= p:
        return np.float32(np.inf)
    while hi - lo > 1:                  # invariant: f(lo) < p <= f(hi)
        mid = (lo + hi) // 2
        if sigmoid_f32(_f32_from_key(mid)) >= p:
            hi = mid
        else:
            lo = mid
    return _f32_from_key(hi)


def predict_mask(h, D, U, b, threshold: float = 0.5):
    """predictor.py:77-79: sigmoid(logits) >= threshold, evaluated in logit
    space in float64."""
    return predictor_logits(h, D, U, b) >= logit_threshold(threshold)


def cold_ids_for(mask_row, hot_ids, inter_dim: int):
    """engine.py:274-283: ascending nonzero ids of the mask minus hot ids; with
    no predictor (mask None) every non-hot id in range(inter_dim)."""
    hot = set(int(i) for i in hot_ids)
    if mask_row is None:
        return [i for i in range(inter_dim) if i not in hot]
    ids = np.nonzero(np.asarray(mask_row))[0].tolist()
    return [i for i in ids if i not in hot]


def query(x_rows_normed_f16):
    """engine.py:277: the predictor query is the mean over the batch of the
    normalised last-token rows.  The rows are fp16 and torch's fp16 mean
    accumulates in fp32 and rounds to fp16."""
    x = np.asarray(x_rows_normed_f16, dtype=np.float16).astype(np.float32)
    acc = np.zeros(x.shape[1], np.float32)
    for row in x:
        acc = acc + row
    return (acc / np.float32(x.shape[0])).astype(np.float16)


def to_bf16(v):
    """Round-to-nearest-even float32 -> bfloat16, returned as float32 values
    (the cast predictor.py:455 applies for a bf16 predictor).  Overflow past
    the largest bfloat16 rounds to infinity; NaN stays NaN (a quiet NaN)."""
    f = np.asarray(v, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    u = np.where(np.isnan(f), np.uint64(0x7FC00000), u)
    return u.astype(np.uint32).view(np.float32)


# ── device-layout helpers: raw bytes -> dense float64 weights ────────────────

def records_to_dense(records, slots, H: int = HIDDEN_DIM):
    """Records (n, 6400) uint8 and a slot list -> (gate (k,H), up (k,H),
    down (H,k)) float64 in slot order, each record decoded by record_vectors."""
    recs = np.asarray(records, dtype=np.uint8)
    g, u, d = [], [], []
    for s in slots:
        buf = recs[int(s)].tobytes()
        _, a, b, c = record_vectors(buf, 0, H)
        g.append(a)
        u.append(b)
        d.append(c)
    if not g:
        z = np.zeros((0, H))
        return z, z, z.T
    return (np.stack(g).astype(np.float64), np.stack(u).astype(np.float64),
            np.stack(d, axis=1).astype(np.float64))


def hot_to_dense(gate_q, up_q, down_q, gate_s, up_s, down_s):
    """fp8 codes with per-row scales -> float64 (n,H), (n,H), (H,n)."""
    return (fp8_dequant(gate_q, gate_s), fp8_dequant(up_q, up_s), fp8_dequant(down_q, down_s))


def rel_err(y, ref):
    """Normwise max relative error max|y - ref| / max|ref|."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    return float(np.abs(y - ref).max() / max(np.abs(ref).max(), 1e-30))


def cosine(y, ref):
    y = np.asarray(y, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    return float(y @ ref / max(np.linalg.norm(y) * np.linalg.norm(ref), 1e-300))


def ambiguous(logits, threshold: float = 0.5, band: float = 1e-6):
    """Neurons whose logit is within ``band`` of the threshold: the parity
    contract exempts these from index-set equality."""
    return np.abs(np.asarray(logits, np.float64) - logit_threshold(threshold)) <= band


# ── attention (engine.py:63-157) ────────────────────────────────────────────

def rope_cache(max_seq_len: int, head_dim: int, theta: float):
    """engine.py:128-137 in float64: angle[t, i] = t * theta^(-i / half) for
    i < half = head_dim // 2; returns (cos, sin), each (max_seq_len, half)."""
    half = head_dim // 2
    inv = 1.0 / (float(theta) ** (np.arange(half, dtype=np.float64) / half))
    ang = np.outer(np.arange(max_seq_len, dtype=np.float64), inv)
    return np.cos(ang), np.sin(ang)


def apply_rope(x, cos, sin):
    """engine.py:140-157: x (..., T, D) split into halves x1 = x[..., :D/2],
    x2 = x[..., D/2:]; returns cat(x1 cos - x2 sin, x1 sin + x2 cos) with the
    tables (T, D/2) broadcast over the leading axes.  The reference casts the
    tables to the activations' dtype first (engine.py:153-154); callers that
    model that pass fp16-rounded tables."""
    x = np.asarray(x, np.float64)
    half = x.shape[-1] // 2
    c = np.asarray(cos, np.float64)
    s = np.asarray(sin, np.float64)
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x1 * s + x2 * c], axis=-1)


def attention_core(q, k, v, causal: bool):
    """F.scaled_dot_product_attention as engine.py:118-121 calls it, after
    repeat_interleave of the kv heads (engine.py:114-116): q (B, n_q, T, D),
    k/v (B, n_kv, S, D); query head h reads kv head h // (n_q // n_kv);
    scores scaled by 1/sqrt(D); with ``causal`` query t sees keys
    s <= t (torch's top-left alignment, which the engine only uses with
    T == S); float64."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, n_q, T, D = q.shape
    n_kv, S = k.shape[1], k.shape[2]
    grp = n_q // n_kv
    kk = np.repeat(k, grp, axis=1)
    vv = np.repeat(v, grp, axis=1)
    sc = q @ np.swapaxes(kk, -1, -2) / math.sqrt(D)
    if causal:
        mask = np.arange(S)[None, :] > np.arange(T)[:, None]
        sc = np.where(mask, -np.inf, sc)
    sc = sc - sc.max(axis=-1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(axis=-1, keepdims=True)
    return p @ vv


def f16(v):
    """Round to fp16 and back to float64 (the reference's fp16 activations)."""
    return np.asarray(v, np.float64).astype(np.float16).astype(np.float64)


def gqa_attention(x, norm_w, eps, wq, wk, wv, wo, n_q, n_kv, cos, sin, kv_cache=None):
    """GroupedQueryAttention.forward (engine.py:90-125) in float64 with the
    reference's fp16 rounding points: x_n = fp16(RMSNorm(x)) (engine.py:93,
    nn.RMSNorm on fp16); q, k, v = fp16(x_n W^T) (:94-96); RoPE with the
    tables rounded to fp16 and its result rounded to fp16 (:102-103,
    :153-157); k, v appended to the cache (:105-109); attention of every query
    over the cache, causal only without a cache (:118-121), rounded to fp16;
    out = fp16(attn W_o^T) (:122-123).
    x (B, T, H); weights dense (out, in); cos/sin (T, D/2) for the call's
    positions; kv_cache None or (k (B, n_kv, S, D), v).  Returns
    (out (B, T, H), (k, v) with S + T positions)."""
    x = np.asarray(x, np.float64)
    B, T, H = x.shape
    D = H // n_q
    xn = f16(rmsnorm(x, norm_w, eps))
    q = f16(xn @ np.asarray(wq, np.float64).T).reshape(B, T, n_q, D).transpose(0, 2, 1, 3)
    k = f16(xn @ np.asarray(wk, np.float64).T).reshape(B, T, n_kv, D).transpose(0, 2, 1, 3)
    v = f16(xn @ np.asarray(wv, np.float64).T).reshape(B, T, n_kv, D).transpose(0, 2, 1, 3)
    c16, s16 = f16(cos)[:T], f16(sin)[:T]
    q = f16(apply_rope(q, c16, s16))
    k = f16(apply_rope(k, c16, s16))
    if kv_cache is not None:
        k = np.concatenate([np.asarray(kv_cache[0], np.float64), k], axis=2)
        v = np.concatenate([np.asarray(kv_cache[1], np.float64), v], axis=2)
    o = f16(attention_core(q, k, v, causal=kv_cache is None))
    o = o.transpose(0, 2, 1, 3).reshape(B, T, n_q * D)
    return f16(o @ np.asarray(wo, np.float64).T), (k, v)
