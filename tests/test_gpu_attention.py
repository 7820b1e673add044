"""GPU parity of the decode attention (oi2_attn_forward through
oi2.GroupedQueryAttention) against the oracle's restatement of
GroupedQueryAttention.forward (engine.py:90-125).

Bar: the attention output (o_proj, fp16) and the new cache rows within max
rel err 1e-2 and cosine >= 0.9999 of the float64 oracle over the same fp8
weights and the same cache contents; cache positions below ``past`` are left
bit for bit; the fused residual is exactly fp16(x + out).
"""
import numpy as np
import pytest
import torch

import oi2
from oracle import oracle as O
from tests.gpu_helpers import EPS, assert_ffn_close

pytestmark = pytest.mark.gpu
H = 4096
D = 128


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


def _weights(dev, n_kv, seed, layer=0):
    """A shared-weights dict as splitter.py:175-179 writes it: fp8 e4m3fn
    projections, fp16 input_layernorm."""
    g = torch.Generator(device=dev).manual_seed(seed)
    n_q = H // D

    def w(rows, cols):
        return (torch.randn((rows, cols), generator=g, device=dev) * 0.02).to(torch.float8_e4m3fn)

    p = f"layer_{layer:03d}."
    return {p + "q_proj": w(n_q * D, H), p + "k_proj": w(n_kv * D, H), p + "v_proj": w(n_kv * D, H),
            p + "o_proj": w(H, n_q * D),
            p + "input_layernorm": (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).half()}


def _cfg(n_kv):
    return {"num_attention_heads": H // D, "num_key_value_heads": n_kv, "hidden_dim": H,
            "rms_norm_eps": EPS}


def _dense(weights, layer=0):
    p = f"layer_{layer:03d}."
    f = lambda n: weights[p + n].float().cpu().numpy().astype(np.float64)
    return (f("q_proj"), f("k_proj"), f("v_proj"), f("o_proj"),
            weights[p + "input_layernorm"].float().cpu().numpy().astype(np.float64))


def _oracle(weights, n_kv, x, cos, sin, cache):
    wq, wk, wv, wo, nw = _dense(weights)
    kv = None if cache is None else (cache[0].float().cpu().numpy(), cache[1].float().cpu().numpy())
    T = x.shape[1]
    return O.gqa_attention(x.float().cpu().numpy(), nw, EPS, wq, wk, wv, wo, H // D, n_kv,
                           cos[:T].cpu().numpy(), sin[:T].cpu().numpy(), kv)


def _check_step(attn, weights, n_kv, x, cos, sin, cache, what):
    """One call against the oracle over the same cache contents; returns the
    call's (out, (k, v))."""
    before = None if cache is None else (cache[0].clone(), cache[1].clone())
    res = torch.empty_like(x)
    out, (k, v) = attn(x, cos, sin, cache, residual_out=res)
    torch.cuda.synchronize()
    ref, (rk, rv) = _oracle(weights, n_kv, x, cos, sin, before)
    print(f"[attn] {what}: out {tuple(out.shape)}, cache {tuple(k.shape)}", flush=True)
    assert_ffn_close(out.float().cpu().numpy(), ref, what=f"{what} out")
    past = 0 if before is None else before[0].shape[2]
    T = x.shape[1]
    assert k.shape == (x.shape[0], n_kv, past + T, D) and v.shape == k.shape
    assert_ffn_close(k[:, :, past:].float().cpu().numpy(), rk[:, :, past:], what=f"{what} new k")
    assert_ffn_close(v[:, :, past:].float().cpu().numpy(), rv[:, :, past:], what=f"{what} new v")
    if before is not None:
        assert torch.equal(k[:, :, :past], before[0]) and torch.equal(v[:, :, :past], before[1])
    assert torch.equal(res, (x.float() + out.float()).half()), f"{what}: fused residual"
    return out, (k, v)


def _rand_cache(dev, B, n_kv, past, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn((B, n_kv, past, D), generator=g, device=dev).half()
    v = torch.randn((B, n_kv, past, D), generator=g, device=dev).half()
    return k, v


@pytest.mark.parametrize("B,past,n_kv", [(1, 5, 8), (1, 37, 8), (3, 300, 8), (1, 4095, 8), (3, 1000, 8), (2, 100, 32),
                                         (2, 129, 4), (1, 255, 16), (1, 1023, 8), (2, 1024, 8)])
def test_decode_step_against_oracle(dev, B, past, n_kv):
    """One token per sequence over a cache from elsewhere (copied into the
    layer's buffer): query groups of 1, 2, 4, 8; spans up to 1024 positions
    in one workgroup per query head (1024 itself included), longer ones split
    over the sequence (1025 and 4096 positions)."""
    w = _weights(dev, n_kv, seed=past + n_kv)
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(past + 8, D, 10000.0, device=dev)
    g = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn((B, 1, H), generator=g, device=dev).half()
    cache = _rand_cache(dev, B, n_kv, past, seed=past)
    _check_step(attn, w, n_kv, x, cos[past:], sin[past:], cache, f"decode B={B} past={past} n_kv={n_kv}")


def test_prefill_then_decode_like_the_engine(dev):
    """engine.py:406-442's use: a causal prefill without a cache, then
    decode steps that pass back the cache the previous call returned (the
    in-place append), each checked over the cache it was given; the RoPE
    positions continue from the cache length (engine.py:414-416)."""
    n_kv, B, T = 8, 2, 5
    w = _weights(dev, n_kv, seed=11)
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(64, D, 1e6, device=dev)
    g = torch.Generator(device=dev).manual_seed(12)
    x = torch.randn((B, T, H), generator=g, device=dev).half()
    _, kv = _check_step(attn, w, n_kv, x, cos, sin, None, "prefill B=2 T=5")
    ptr = kv[0].data_ptr()
    for step in range(3):
        past = kv[0].shape[2]
        xt = torch.randn((B, 1, H), generator=g, device=dev).half()
        _, kv = _check_step(attn, w, n_kv, xt, cos[past:past + 1], sin[past:past + 1], kv,
                            f"decode step {step}")
        assert kv[0].data_ptr() == ptr, "the returned cache is appended in place"


def test_rows_beyond_one_launch_and_noncausal_chunk(dev):
    """12 query rows (two projection launches of up to 8 rows), causal
    prefill; then a 3-token chunk over a cache, which the reference runs
    non-causally (is_causal is False whenever a cache is given,
    engine.py:121)."""
    n_kv, B = 8, 3
    w = _weights(dev, n_kv, seed=21)
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(64, D, 10000.0, device=dev)
    g = torch.Generator(device=dev).manual_seed(22)
    x = torch.randn((B, 4, H), generator=g, device=dev).half()
    _, kv = _check_step(attn, w, n_kv, x, cos, sin, None, "prefill B=3 T=4")
    x2 = torch.randn((B, 3, H), generator=g, device=dev).half()
    _check_step(attn, w, n_kv, x2, cos[4:], sin[4:], kv, "chunk of 3 over a cache")


def test_cache_growth_and_default_norm(dev):
    """A decode past the buffer's room moves the cache to a larger buffer
    with its contents; a weights dict without input_layernorm uses
    nn.RMSNorm's default weight of ones (engine.py:85-88)."""
    n_kv, B = 8, 1
    w = _weights(dev, n_kv, seed=31)
    del w["layer_000.input_layernorm"]
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(300, D, 10000.0, device=dev)
    g = torch.Generator(device=dev).manual_seed(32)
    x = torch.randn((B, 255, H), generator=g, device=dev).half()
    _, kv = attn(x, cos, sin)
    assert attn.capacity == 256
    w["layer_000.input_layernorm"] = torch.ones(H, dtype=torch.float16, device=dev)
    for step in range(2):
        past = kv[0].shape[2]
        xt = torch.randn((B, 1, H), generator=g, device=dev).half()
        _, kv = _check_step(attn, w, n_kv, xt, cos[past:], sin[past:], kv, f"growth step {step}")
    assert attn.capacity == 512 and kv[0].shape[2] == 257


def test_returned_caches_never_change(dev):
    """Tensors a call returned keep their contents whatever later calls do:
    a second sequence (kv_cache=None), a roll-back to an older, shorter view
    of the cache, and the in-place append of the latest view (which writes
    only past the earlier views' ends).  The reference returns fresh
    torch.cat tensors every call (engine.py:105-109)."""
    n_kv, B = 8, 1
    w = _weights(dev, n_kv, seed=41)
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(64, D, 10000.0, device=dev)
    g = torch.Generator(device=dev).manual_seed(42)
    x = torch.randn((B, 6, H), generator=g, device=dev).half()
    _, kv_a = attn(x, cos, sin)
    xt = torch.randn((B, 1, H), generator=g, device=dev).half()
    _, kv_a1 = attn(xt, cos[6:], sin[6:], kv_a)          # in place: kv_a is unchanged
    torch.cuda.synchronize()
    snap = [t.clone() for t in (*kv_a, *kv_a1)]
    x2 = torch.randn((B, 9, H), generator=g, device=dev).half()
    _, kv_b = attn(x2, cos, sin)                          # a second sequence
    x3 = torch.randn((B, 1, H), generator=g, device=dev).half()
    _, kv_r = _check_step(attn, w, n_kv, x3, cos[6:], sin[6:], kv_a, "roll back to 6 positions")
    torch.cuda.synchronize()
    for t, s in zip((*kv_a, *kv_a1), snap):
        assert torch.equal(t, s), "a returned cache changed"
    assert kv_b[0].shape[2] == 9 and kv_r[0].shape[2] == 7
    assert kv_b[0].data_ptr() != kv_a[0].data_ptr() and kv_r[0].data_ptr() != kv_a[0].data_ptr()
    # the roll-back's new position differs from the first sequence's own 7th
    assert not torch.equal(kv_r[0][:, :, 6], kv_a1[0][:, :, 6])


def test_rewind_decodes_a_position_again_in_place(dev):
    """rewind(n) is the one opt-in roll-back that reuses the buffer: a view
    of length n then appends in place at position n, the first n positions
    stay bit for bit, and decoding the same token at the same position twice
    gives the same output and cache row (the oracle checks the step)."""
    n_kv, B = 8, 1
    w = _weights(dev, n_kv, seed=43)
    attn = oi2.GroupedQueryAttention(0, w, _cfg(n_kv))
    cos, sin = oi2.rope_tables(64, D, 10000.0, device=dev)
    g = torch.Generator(device=dev).manual_seed(44)
    x = torch.randn((B, 10, H), generator=g, device=dev).half()
    _, kv = attn(x, cos, sin)
    view = (kv[0][:, :, :10], kv[1][:, :, :10])
    head = [t.clone() for t in view]
    xt = torch.randn((B, 1, H), generator=g, device=dev).half()
    out1, kv1 = _check_step(attn, w, n_kv, xt, cos[10:], sin[10:], view, "decode at 10")
    row1 = (kv1[0][:, :, 10].clone(), kv1[1][:, :, 10].clone())
    attn.rewind(10)
    out2, kv2 = attn(xt, cos[10:], sin[10:], view)
    torch.cuda.synchronize()
    assert kv2[0].data_ptr() == kv[0].data_ptr(), "rewind must reuse the layer's buffer"
    assert torch.equal(out1, out2)
    assert torch.equal(kv2[0][:, :, 10], row1[0]) and torch.equal(kv2[1][:, :, 10], row1[1])
    for t, s in zip(view, head):
        assert torch.equal(t, s)
    with pytest.raises(ValueError):
        attn.rewind(12)
