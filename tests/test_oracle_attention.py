"""Pins for the oracle's attention restatement (engine.py:63-157): closed
forms of the RoPE table, invariants of the rotation, torch's own
scaled_dot_product_attention as the library routine, and the decode step
against the last row of a causal prefill."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O


def test_rope_cache_closed_form():
    cos, sin = O.rope_cache(64, 128, 10000.0)
    assert cos.shape == sin.shape == (64, 64)
    assert np.allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-15)
    assert np.array_equal(cos[0], np.ones(64)) and np.array_equal(sin[0], np.zeros(64))
    # i = 0 rotates by t radians; i = half/2 by t * theta^(-1/2) = t / 100
    t = np.arange(64)
    assert np.allclose(cos[:, 0], np.cos(t), atol=1e-15)
    assert np.allclose(sin[:, 32], np.sin(t / 100.0), atol=1e-15)
    # the last frequency is theta^(-(half-1)/half)
    assert np.allclose(sin[:, 63], np.sin(t * 10000.0 ** (-63 / 64)), atol=1e-15)
    # torch's float32 table (engine.py:128-137 computes it in float32) agrees
    # with the float64 one to float32 precision of the angle
    half = 64
    freqs = 1.0 / (10000.0 ** (torch.arange(0, half).float() / half))
    ang = torch.outer(torch.arange(64).float(), freqs)
    assert np.allclose(ang.cos().numpy(), cos, atol=5e-5)


def test_apply_rope_convention_and_invariants():
    rng = np.random.default_rng(0)
    D, half = 128, 64
    cos, sin = O.rope_cache(40, D, 10000.0)
    # the half-split convention and its signs: e_0 -> (cos, +sin at half),
    # e_half -> (-sin at 0, cos at half)
    for p in (1, 7, 33):
        e0 = np.zeros(D)
        e0[0] = 1
        r = O.apply_rope(e0[None], cos[p:p + 1], sin[p:p + 1])[0]
        assert np.isclose(r[0], cos[p, 0]) and np.isclose(r[half], sin[p, 0])
        assert np.count_nonzero(r) == 2
        eh = np.zeros(D)
        eh[half] = 1
        r = O.apply_rope(eh[None], cos[p:p + 1], sin[p:p + 1])[0]
        assert np.isclose(r[0], -sin[p, 0]) and np.isclose(r[half], cos[p, 0])
    x = rng.standard_normal((3, 40, D))
    # position 0 is the identity
    assert np.allclose(O.apply_rope(x[:, :1], cos[:1], sin[:1]), x[:, :1])
    y = O.apply_rope(x, cos, sin)
    # every (i, i + half) pair keeps its norm
    assert np.allclose(x[..., :half] ** 2 + x[..., half:] ** 2, y[..., :half] ** 2 + y[..., half:] ** 2)
    # the dot of q at m and k at n depends on m - n only
    q, k = rng.standard_normal(D), rng.standard_normal(D)
    def rot(v, p):
        return O.apply_rope(v[None], cos[p:p + 1], sin[p:p + 1])[0]
    for m, n, d in ((5, 2, 11), (30, 30, 4), (0, 9, 20)):
        assert np.isclose(rot(q, m) @ rot(k, n), rot(q, m + d) @ rot(k, n + d))
    # rotating by p1 then p2 is rotating by p1 + p2
    assert np.allclose(rot(rot(q, 6), 13), rot(q, 19))


def _sdpa_torch(q, k, v, causal):
    return F.scaled_dot_product_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                          is_causal=causal, enable_gqa=True).numpy()


@pytest.mark.parametrize("n_q,n_kv,T,S,causal", [(8, 2, 1, 37, False), (8, 8, 3, 19, False),
                                                  (32, 8, 5, 5, True), (4, 1, 9, 9, True)])
def test_attention_core_matches_torch_sdpa(n_q, n_kv, T, S, causal):
    rng = np.random.default_rng(n_q + 3 * T)
    q = rng.standard_normal((2, n_q, T, 128))
    k = rng.standard_normal((2, n_kv, S, 128))
    v = rng.standard_normal((2, n_kv, S, 128))
    got = O.attention_core(q, k, v, causal)
    want = _sdpa_torch(q, k, v, causal)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_attention_core_special_cases():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 4, 1, 128))
    v = rng.standard_normal((1, 2, 1, 128))
    k = rng.standard_normal((1, 2, 1, 128))
    # one key: every query head returns its group's value
    out = O.attention_core(q, k, v, False)
    assert np.allclose(out[0, 0, 0], v[0, 0, 0]) and np.allclose(out[0, 1, 0], v[0, 0, 0])
    assert np.allclose(out[0, 2, 0], v[0, 1, 0]) and np.allclose(out[0, 3, 0], v[0, 1, 0])
    # equal keys: the mean of the values
    k = np.repeat(rng.standard_normal((1, 2, 1, 128)), 6, axis=2)
    v = rng.standard_normal((1, 2, 6, 128))
    out = O.attention_core(q, k, v, False)
    assert np.allclose(out[0, 3, 0], v[0, 1].mean(0))


def _layer(rng, n_q, n_kv, H=4096):
    D = H // n_q
    s = 0.02
    return (rng.standard_normal((n_q * D, H)) * s, rng.standard_normal((n_kv * D, H)) * s,
            rng.standard_normal((n_kv * D, H)) * s, rng.standard_normal((H, n_q * D)) * s,
            1.0 + 0.1 * rng.standard_normal(H))


def test_gqa_single_token_returns_grouped_values():
    """With no cache and one token, attention returns each query head its
    group's value, so out = fp16(fp16(v-heads repeated) W_o^T): pins the value
    path, the head layout and the repeat_interleave grouping (engine.py:114-116),
    which a tiled grouping would get wrong."""
    rng = np.random.default_rng(1)
    n_q, n_kv = 32, 8
    wq, wk, wv, wo, nw = _layer(rng, n_q, n_kv)
    x = rng.standard_normal((2, 1, 4096))
    cos, sin = O.rope_cache(4, 128, 10000.0)
    out, (k, v) = O.gqa_attention(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[:1], sin[:1])
    xn = O.f16(O.rmsnorm(x, nw, 1e-5))
    vv = O.f16(xn @ wv.T).reshape(2, 1, n_kv, 128)
    heads = np.repeat(vv, n_q // n_kv, axis=2).reshape(2, 1, 4096)
    assert np.allclose(out, O.f16(heads @ wo.T), rtol=0, atol=0)
    assert k.shape == v.shape == (2, n_kv, 1, 128)
    assert np.array_equal(v[:, :, 0, :], vv[:, 0])


def test_gqa_decode_equals_last_row_of_causal_prefill():
    """A prefill of T tokens, then one decode step with that cache, gives the
    same last row as a causal prefill of T + 1 tokens (engine.py:118-121: the
    decode step attends to the whole cache, the prefill causally)."""
    rng = np.random.default_rng(2)
    n_q, n_kv, T = 32, 8, 6
    wq, wk, wv, wo, nw = _layer(rng, n_q, n_kv)
    x = rng.standard_normal((1, T + 1, 4096))
    cos, sin = O.rope_cache(T + 1, 128, 10000.0)
    full, (kf, vf) = O.gqa_attention(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos, sin)
    _, kv = O.gqa_attention(x[:, :T], nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[:T], sin[:T])
    last, (k2, v2) = O.gqa_attention(x[:, T:], nw, 1e-5, wq, wk, wv, wo, n_q, n_kv,
                                     cos[T:], sin[T:], kv_cache=kv)
    assert np.array_equal(last[0, 0], full[0, T])
    assert np.array_equal(k2, kf) and np.array_equal(v2, vf)
    # the earlier rows do differ from a non-causal pass, so causality is real
    nc = O.attention_core(np.ones((1, 1, 2, 4)), np.array([[[[0, 0, 0, 0], [5, 5, 5, 5]]]], float),
                          np.array([[[[1, 1, 1, 1], [2, 2, 2, 2]]]], float), causal=True)
    assert np.allclose(nc[0, 0, 0], 1.0)


def test_gqa_relative_positions_and_rope_only_on_q_k():
    """Shifting every position by the same offset changes nothing but
    rounding: RoPE enters only through q . k (engine.py:102-103), never v."""
    rng = np.random.default_rng(5)
    n_q, n_kv, T = 8, 2, 5
    H = 1024
    wq, wk, wv, wo, nw = _layer(rng, n_q, n_kv, H)
    x = rng.standard_normal((1, T, H))
    cos, sin = O.rope_cache(T + 50, H // n_q, 10000.0)
    a, _ = O.gqa_attention(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[:T], sin[:T])
    b, _ = O.gqa_attention(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[50:], sin[50:])
    # (a rotation applied to v as well would move the output with the shift)
    assert O.rel_err(b, a) < 1e-2 and O.cosine(b, a) > 0.9999


def _torch_gqa(x, nw, eps, wq, wk, wv, wo, n_q, n_kv, cos, sin, kv_cache, head_split="reference"):
    """GroupedQueryAttention.forward (engine.py:90-125) composed from torch's
    own modules in float64, with the reference's fp16 rounding points as
    casts: nn.RMSNorm, F.linear, view(B, T, n, D).transpose(1, 2), the
    half-split rotation with fp16 tables, torch.cat onto the cache,
    repeat_interleave over the kv heads, scaled_dot_product_attention
    (causal only without a cache), transpose back and o_proj.
    head_split="wrong" splits the heads as view(B, n, T, D) instead (a
    plausible mistake the comparison must catch)."""
    r = lambda t: t.half().double()
    t64 = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    x = t64(x)
    B, T, H = x.shape
    D = H // n_q
    norm = torch.nn.RMSNorm(H, eps=eps, dtype=torch.float64)
    with torch.no_grad():
        norm.weight.copy_(t64(nw))
        xn = r(norm(x))

    def heads(t, n):
        if head_split == "wrong":
            return t.reshape(B, n, T, D)
        return t.view(B, T, n, D).transpose(1, 2)

    q = heads(r(F.linear(xn, t64(wq))), n_q)
    k = heads(r(F.linear(xn, t64(wk))), n_kv)
    v = heads(r(F.linear(xn, t64(wv))), n_kv)

    def rope(t):
        half = D // 2
        c = r(t64(cos)[:T])[None, None]
        s = r(t64(sin)[:T])[None, None]
        a, b = t[..., :half], t[..., half:]
        return r(torch.cat([a * c - b * s, a * s + b * c], dim=-1))

    q, k = rope(q), rope(k)
    if kv_cache is not None:
        k = torch.cat([t64(kv_cache[0]), k], dim=2)
        v = torch.cat([t64(kv_cache[1]), v], dim=2)
    g = n_q // n_kv
    o = F.scaled_dot_product_attention(q, k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1),
                                       is_causal=kv_cache is None)
    o = r(o).transpose(1, 2).contiguous().view(B, T, H)
    return r(F.linear(o, t64(wo))).numpy(), (k.numpy(), v.numpy())


@pytest.mark.parametrize("n_q,n_kv,H,T,past", [(32, 8, 4096, 4, 0), (32, 8, 4096, 1, 23),
                                               (8, 2, 1024, 5, 0), (8, 2, 1024, 2, 11)])
def test_gqa_matches_torch_composition(n_q, n_kv, H, T, past):
    """The oracle's attention against the torch composition of engine.py:90-125
    with the same rounding points, with and without a cache; the head split,
    the kv grouping, the rotation and the cache order all enter the result.
    A wrong head split in the composition is far from the oracle, so the
    comparison would catch that mistake on either side."""
    rng = np.random.default_rng(100 + n_q + T + past)
    wq, wk, wv, wo, nw = _layer(rng, n_q, n_kv, H)
    D = H // n_q
    x = rng.standard_normal((2, T, H))
    cos, sin = O.rope_cache(past + T, D, 10000.0)
    cache = None
    if past:
        cache = (O.f16(rng.standard_normal((2, n_kv, past, D))), O.f16(rng.standard_normal((2, n_kv, past, D))))
    got, (gk, gv) = O.gqa_attention(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[past:], sin[past:], cache)
    want, (wk2, wv2) = _torch_gqa(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[past:], sin[past:], cache)
    assert got.shape == want.shape == (2, T, H)
    # fp16 rounding points may flip by one ulp where float64 sums differ in order
    assert O.rel_err(got, want) < 2e-3 and O.cosine(got, want) > 0.99999
    assert O.rel_err(gk, wk2) < 2e-3 and O.rel_err(gv, wv2) < 2e-3
    bad, _ = _torch_gqa(x, nw, 1e-5, wq, wk, wv, wo, n_q, n_kv, cos[past:], sin[past:], cache, head_split="wrong")
    if T > 1:
        assert O.rel_err(bad, want) > 0.05, "a wrong head split must be visible"
