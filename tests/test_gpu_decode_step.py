"""GPU tests of the decode step composed from the drop-in layers
(oi2.DecoderStep over GroupedQueryAttention and SparseFFNLayer), built from
split files the way DesdemonaEngine builds its layers (engine.py:384-398).

The reference predicts each layer's cold set ahead of time (its "lookahead
approximation", engine.py:421-436): layer 0's from the embedded tokens, layer
l+1's from layer l's post-attention state, before layer l's FFN has run.

* The step equals a plain loop of the same layers that makes each prediction
  from those same states but only just before the layer's FFN, bit for bit:
  the order in which the step enqueues the work changes nothing (every kernel
  up to 16 tokens adds its partial sums in a fixed order).
* The step's output is within the FFN bar (max rel err 1e-2, cosine >= 0.9999)
  of the oracle's chain: attention (engine.py:90-125), fp16 residual
  (engine.py:426-427), the sparse FFN over the cold set the device selected
  and fp16 residual (engine.py:292-312), layer after layer.  The selection
  itself is pinned by the predictor tests.
* A graph-captured step replayed several times, with eager work and
  synchronisations between the replays, equals the eager step every time.
"""
import os
import tempfile

import numpy as np
import pytest
import torch

import oi2
from oi2.decode_step import DecoderStep
from oi2.layer import rmsnorm
from oi2.synth import SyntheticLayer
from oracle import oracle as O
from tests.gpu_helpers import EPS, assert_ffn_close, cold_dense, hot_dense, normed_f16

pytestmark = pytest.mark.gpu
H = 4096
D = 128
INTER = 14336
N_KV = 8


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


def _attn_weights(g, dev, n_layers):
    w = {}
    for li in range(n_layers):
        p = f"layer_{li:03d}."

        def m(r, c):
            return (torch.randn((r, c), generator=g, device=dev) * 0.02).to(torch.float8_e4m3fn)
        w.update({p + "q_proj": m(H, H), p + "k_proj": m(N_KV * D, H), p + "v_proj": m(N_KV * D, H),
                  p + "o_proj": m(H, H),
                  p + "input_layernorm": (1.0 + 0.1 * torch.randn(H, generator=g, device=dev)).half()})
    return w


@pytest.fixture(scope="module")
def split(dev):
    """Two layers written as the splitter lays them out: hot .pt files, one
    cold file, fp32 predictor files; plus the shared attention weights."""
    n_layers = 2
    g = torch.Generator(device=dev).manual_seed(61)
    syn = [SyntheticLayer(g, INTER, 3584, device=dev, with_predictor=True, pred_dtype=torch.float32)
           for _ in range(n_layers)]
    attn_w = _attn_weights(g, dev, n_layers)
    tmp = tempfile.TemporaryDirectory(dir=os.path.dirname(os.path.abspath(__file__)))
    hot_dir, pdir = os.path.join(tmp.name, "hot"), os.path.join(tmp.name, "pred")
    os.makedirs(hot_dir)
    os.makedirs(pdir)
    w = oi2.format.ColdFileWriter(os.path.join(tmp.name, "cold_weights.bin"), n_layers)
    for li, lay in enumerate(syn):
        lay.hot.save(os.path.join(hot_dir, f"layer_{li:03d}_expert_000.pt"))
        lay.predictor.save(os.path.join(pdir, f"layer_{li:03d}_expert_000.pt"))
        w.add_section(li, lay.records.cpu().numpy())
    w.close(os.path.join(tmp.name, "cold_index.npy"))
    cfg = {"hidden_dim": H, "intermediate_dim": INTER, "hidden_act": "silu", "act_on_both": False,
           "rms_norm_eps": EPS, "num_experts": 1, "num_attention_heads": H // D,
           "num_key_value_heads": N_KV}
    store = oi2.ColdWeightStore(os.path.join(tmp.name, "cold_weights.bin"),
                                os.path.join(tmp.name, "cold_index.npy"), cfg, device=dev)
    reg = oi2.PredictorRegistry(pdir, device=dev)
    yield {"syn": syn, "attn_w": attn_w, "cfg": cfg, "store": store, "reg": reg, "hot_dir": hot_dir,
           "n_layers": n_layers}
    store.close()
    tmp.cleanup()


def _layers(split, dev):
    cfg = split["cfg"]
    attn = [oi2.GroupedQueryAttention(li, split["attn_w"], cfg) for li in range(split["n_layers"])]
    ffn = [oi2.SparseFFNLayer(li, split["hot_dir"], split["store"], split["reg"], cfg, dev, None,
                              ffn_norm_weight=lay.norm_w.cpu())
           for li, lay in enumerate(split["syn"])]
    return attn, ffn


def _caches(dev, n_layers, B, past, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for _ in range(n_layers):
        k = torch.randn((B, N_KV, past, D), generator=g, device=dev).half()
        out.append((k, torch.randn((B, N_KV, past, D), generator=g, device=dev).half()))
    return out


@pytest.mark.parametrize("B", [1, 2])
def test_step_equals_plain_loop_and_oracle_chain(dev, split, B):
    past = 40
    cos, sin = oi2.rope_tables(past + 1, D, 1e6, device=dev)
    c1, s1 = cos[past:], sin[past:]
    g = torch.Generator(device=dev).manual_seed(62)
    x0 = torch.randn((B, 1, H), generator=g, device=dev).half()
    caches = _caches(dev, split["n_layers"], B, past, seed=63)
    attn, ffn = _layers(split, dev)
    print(f"[decode step] B={B} past={past} layers={split['n_layers']}", flush=True)
    y, kv = DecoderStep(attn, ffn)(x0, c1, s1, caches)

    # the same layers one after the other, each prediction made just before
    # its FFN from the state the reference predicts it from
    attn2, ffn2 = _layers(split, dev)
    x, pred_from = x0, [x0]
    for li in range(split["n_layers"]):
        out, _ = attn2[li](x, c1, s1, caches[li])
        x = (x.float() + out.float()).half()
        pred_from.append(x)
        x = ffn2[li](x, ffn2[li].submit_cold_fetch(pred_from[li]))
    torch.cuda.synchronize()
    x0n = x0.float().cpu().numpy()
    assert torch.equal(y, x), "lookahead step differs from the plain loop"
    for li in range(split["n_layers"]):
        assert kv[li][0].shape == (B, N_KV, past + 1, D)
        assert torch.equal(kv[li][0][:, :, :past], caches[li][0])

    # the oracle's chain over the same weights and caches
    xr = x0.float().cpu().numpy().astype(np.float64)
    for li, lay in enumerate(split["syn"]):
        p = f"layer_{li:03d}."
        f = lambda n: split["attn_w"][p + n].float().cpu().numpy().astype(np.float64)
        kvc = (caches[li][0].float().cpu().numpy(), caches[li][1].float().cpu().numpy())
        a, _ = O.gqa_attention(xr, f("input_layernorm"), EPS, f("q_proj"), f("k_proj"), f("v_proj"),
                               f("o_proj"), H // D, N_KV, c1[:1].cpu().numpy(), s1[:1].cpu().numpy(), kvc)
        xr = O.f16(xr + a)
        # the cold set the device selected, from the state the layer predicts it from
        ids = ffn[li]._cold_ids_for(rmsnorm(pred_from[li], lay.norm_w, EPS))
        sec = split["store"].section(li)
        Gc, Uc, Dc = cold_dense(sec.records, sec.slots_for(ids))
        Gh, Uh, Dh = hot_dense(lay.hot)
        xn = normed_f16(torch.from_numpy(xr.reshape(B, H)), lay.norm_w)
        xr = O.f16(xr + O.sparse_ffn(xn, "silu", False, Gh, Uh, Dh, Gc, Uc, Dc).reshape(B, 1, H))
    assert_ffn_close(y.float().cpu().numpy() - x0n, xr - x0n, what="two-layer step")


def test_graph_replays_equal_the_eager_step(dev, split):
    B, past = 1, 300
    cos, sin = oi2.rope_tables(past + 1, D, 1e6, device=dev)
    c1, s1 = cos[past:], sin[past:]
    g = torch.Generator(device=dev).manual_seed(64)
    x0 = torch.randn((B, 1, H), generator=g, device=dev).half()
    attn, ffn = _layers(split, dev)
    step = DecoderStep(attn, ffn)
    stream = torch.cuda.Stream(device=dev)
    print(f"[decode step graph] B={B} past={past}", flush=True)
    with torch.cuda.stream(stream):
        _, kv = step(x0, c1, s1, _caches(dev, split["n_layers"], B, past, seed=65))
        views = [(k[:, :, :past], v[:, :, :past]) for k, v in kv]     # this layer's buffers
        y_eager, _ = step(x0, c1, s1, views)
        y_eager = y_eager.clone()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y, _ = step(x0, c1, s1, views)
    other = torch.randn((512, 512), generator=g, device=dev)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), f"replay {r} differs from the eager step"
        other = (other @ other).tanh()          # eager work between the replays
        torch.cuda.synchronize()
    del graph


def _stack(split):
    """The same layers held by a DecodeStack (its records and LUT from the
    split file's store, the predictors from the registry, threshold 0.5 =
    logit 0)."""
    from oi2.stack import DecodeStack, StackLayer
    layers = []
    for li, lay in enumerate(split["syn"]):
        sec = split["store"].section(li)
        layers.append(StackLayer(lay.hot, sec.records, sec.lut, lay.norm_w, split["reg"].predictors[(li, 0)]))
    return DecodeStack(layers, INTER, EPS, "silu", False, 0.0)


def test_stack_layers_equal_drop_in_layers(dev, split):
    """DecoderStep over a DecodeStack (each layer's FFN and the next layer's
    prediction in two kernels, oi2_stack_layer) against DecoderStep over the
    drop-in SparseFFNLayers: the same output and caches, bit for bit."""
    past = 40
    cos, sin = oi2.rope_tables(past + 1, D, 1e6, device=dev)
    c1, s1 = cos[past:], sin[past:]
    g = torch.Generator(device=dev).manual_seed(66)
    x0 = torch.randn((1, 1, H), generator=g, device=dev).half()
    caches = _caches(dev, split["n_layers"], 1, past, seed=67)
    attn, ffn = _layers(split, dev)
    print("[decode step] drop-in layers vs stack layers", flush=True)
    y_ref, kv_ref = DecoderStep(attn, ffn)(x0, c1, s1, caches)
    attn2, _ = _layers(split, dev)
    stack = _stack(split)
    y, kv = DecoderStep(attn2, stack)(x0, c1, s1, caches)
    torch.cuda.synchronize()
    assert torch.equal(y, y_ref), "stack path differs from the drop-in layers"
    for (k, v), (kr, vr) in zip(kv, kv_ref):
        assert torch.equal(k, kr) and torch.equal(v, vr)
    with pytest.raises(ValueError):
        DecoderStep(attn2, stack)(torch.zeros((2, 1, H), dtype=torch.float16, device=dev), c1, s1, caches)
    stack.close()


def test_stack_step_graph_replays(dev, split):
    """The stack path captured in a graph: every replay equals the eager step."""
    past = 200
    cos, sin = oi2.rope_tables(past + 1, D, 1e6, device=dev)
    c1, s1 = cos[past:], sin[past:]
    g = torch.Generator(device=dev).manual_seed(68)
    x0 = torch.randn((1, 1, H), generator=g, device=dev).half()
    attn, _ = _layers(split, dev)
    stack = _stack(split)
    step = DecoderStep(attn, stack)
    stream = torch.cuda.Stream(device=dev)
    print("[decode step graph] stack layers", flush=True)
    with torch.cuda.stream(stream):
        _, kv = step(x0, c1, s1, _caches(dev, split["n_layers"], 1, past, seed=69))
        views = [(k[:, :, :past], v[:, :, :past]) for k, v in kv]
        y_eager, _ = step(x0, c1, s1, views)
        y_eager = y_eager.clone()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        y, _ = step(x0, c1, s1, views)
    other = torch.randn((512, 512), generator=g, device=dev)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, y_eager), f"replay {r} differs from the eager step"
        other = (other @ other).tanh()
        torch.cuda.synchronize()
    del graph
    stack.close()
