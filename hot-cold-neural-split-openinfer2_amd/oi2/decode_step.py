"""The layer loop of DesdemonaEngine.forward (engine.py:406-442) over this
library's drop-in layers: per layer the attention with its residual
(engine.py:426-427), the next layer's cold fetch submitted from the
post-attention state (the lookahead, engine.py:431-436), then this layer's
FFN with the fetch it was given (engine.py:438).

Embedding, final norm and lm_head stay with the caller, as they are outside
the decode path this library replaces.  With the cold records resident in
HBM (or pinned memory) nothing in the loop waits on the host, so a caller may
capture a whole step in a CUDA/HIP graph.

The FFN side is either the drop-in layers (a list of SparseFFNLayer, any
batch) or a DecodeStack holding the same layers (one token): the stack runs
each layer as two kernels that also predict the next layer's cold set from
the layer's post-attention input, where the drop-in layers run a separate
predictor first.  Both give the same values.
"""
from __future__ import annotations

import torch

from .attention import GroupedQueryAttention
from .layer import SparseFFNLayer
from .stack import DecodeStack


class DecoderStep:
    def __init__(self, attention_layers: list[GroupedQueryAttention],
                 ffn_layers: "list[SparseFFNLayer] | DecodeStack"):
        n_ffn = ffn_layers.n_layers if isinstance(ffn_layers, DecodeStack) else len(ffn_layers)
        if len(attention_layers) != n_ffn:
            raise ValueError(f"{len(attention_layers)} attention layers but {n_ffn} FFN layers")
        self.attention_layers = attention_layers
        self.ffn_layers = ffn_layers

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, kv_caches=None):
        """x (B, T, H) fp16 (the embedded tokens); cos / sin the tables for
        the call's positions; kv_caches None or one (k, v) per layer.
        Returns (x after the last layer's FFN, the new caches), as the loop
        of engine.py:421-438 leaves them before the final norm."""
        if isinstance(self.ffn_layers, DecodeStack):
            return self._forward_stack(x, cos, sin, kv_caches)
        new_kv = []
        B, T, H = x.shape
        next_prefetch = self.ffn_layers[0].submit_cold_fetch(x)
        for li, (attn, ffn) in enumerate(zip(self.attention_layers, self.ffn_layers)):
            kv = kv_caches[li] if kv_caches else None
            resid = torch.empty_like(x)
            _, layer_kv = attn(x, cos, sin, kv, residual_out=resid)   # x + attention
            x = resid
            new_kv.append(layer_kv)
            this_prefetch = next_prefetch
            next_prefetch = (self.ffn_layers[li + 1].submit_cold_fetch(x)
                             if li + 1 < len(self.ffn_layers) else None)
            x = ffn(x, this_prefetch)
        return x, new_kv

    def _forward_stack(self, x, cos, sin, kv_caches):
        B, T, H = x.shape
        if B * T != 1:
            raise ValueError(f"a DecodeStack runs one token at a time, got batch {B} x {T}")
        stack = self.ffn_layers
        stack.predict(0, x.reshape(H))
        new_kv = []
        for li, attn in enumerate(self.attention_layers):
            kv = kv_caches[li] if kv_caches else None
            resid = torch.empty_like(x)
            _, layer_kv = attn(x, cos, sin, kv, residual_out=resid)   # x + attention
            new_kv.append(layer_kv)
            out = torch.empty_like(x)
            stack.layer(li, resid.reshape(H), out.reshape(H))         # FFN, and layer li + 1's set
            x = out
        return x, new_kv

    __call__ = forward
