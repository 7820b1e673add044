"""Grouped-query attention on liboi2's gfx950 kernels: the drop-in
``GroupedQueryAttention`` of engine.py:63-125.

``GroupedQueryAttention(layer_idx, weights, cfg)`` takes the same shared
weights dict the reference loads from hot_weights/shared.pt
(``layer_XXX.q_proj`` ... fp8 e4m3fn, ``layer_XXX.input_layernorm`` fp16;
splitter.py:175-179) and keeps the projections at fp8 in HBM.
``forward(x, cos, sin, kv_cache=None)`` returns ``(out, (k, v))`` as the
reference does: out (B, T, H) fp16 is o_proj of the attention, before the
engine's residual add; k, v are (B, n_kv, S, 128) fp16 with S = past + T.

The reference grows its cache with torch.cat every step (engine.py:105-109).
Here each layer owns one buffer with room for more positions and returns
views of it; a call that passes back the latest views it returned appends in
place, which leaves every earlier returned view as it was (they end before
the positions written).  Any other cache (kv_cache=None, a cache from
anywhere else, or an older, shorter view of this layer's cache) gets a new
buffer, the older cache copied into it: earlier returned tensors never change.

There is no CPU fallback: without liboi2.so or a GPU every call raises.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

HEAD_DIM = 128


def rope_tables(max_seq_len: int, head_dim: int, theta: float, device="cpu"):
    """float32 cos / sin tables (max_seq_len, head_dim // 2) of the angles
    t * theta^(-i / half), the rotary tables engine.py:128-137 builds and
    slices per call (engine.py:414-416)."""
    half = head_dim // 2
    expo = torch.arange(half, device=device, dtype=torch.float32) / half
    freqs = 1.0 / torch.pow(torch.tensor(float(theta), dtype=torch.float32, device=device), expo)
    ang = torch.arange(max_seq_len, device=device, dtype=torch.float32)[:, None] * freqs[None, :]
    return torch.cos(ang), torch.sin(ang)


def _fp8_bytes(w: torch.Tensor, shape, what: str, device) -> torch.Tensor:
    if w.dtype != torch.float8_e4m3fn:
        raise TypeError(f"{what}: expected the split's fp8 e4m3fn weight (splitter.py:177), got {w.dtype}")
    if tuple(w.shape) != tuple(shape):
        raise ValueError(f"{what}: shape {tuple(w.shape)}, expected {tuple(shape)}")
    return w.to(device).contiguous().view(torch.uint8)


class GroupedQueryAttention(torch.nn.Module):
    """engine.py:63-125 on the GPU: RMSNorm, q/k/v projections, RoPE, KV
    append, grouped attention and o_proj as three HIP kernels."""

    def __init__(self, layer_idx: int, weights: dict, cfg: dict, device=None):
        super().__init__()
        self.layer_idx = layer_idx
        self.n_q = int(cfg["num_attention_heads"])
        self.n_kv = int(cfg["num_key_value_heads"])
        self.hidden = int(cfg["hidden_dim"])
        self.head_dim = self.hidden // self.n_q
        if self.hidden != _lib.HIDDEN or self.head_dim != HEAD_DIM:
            raise ValueError(f"hidden {self.hidden} with {self.n_q} heads: this build serves "
                             f"hidden {_lib.HIDDEN}, head_dim {HEAD_DIM}")
        if self.n_q % self.n_kv or self.n_q // self.n_kv not in (1, 2, 4, 8):
            raise ValueError(f"{self.n_q} query heads over {self.n_kv} kv heads: groups of 1, 2, 4 or 8")
        self.eps = float(cfg["rms_norm_eps"])
        prefix = f"layer_{layer_idx:03d}."
        dev = torch.device(device) if device is not None else weights[prefix + "q_proj"].device
        self.device = dev
        qd, kvd = self.n_q * HEAD_DIM, self.n_kv * HEAD_DIM
        self.wq = _fp8_bytes(weights[prefix + "q_proj"], (qd, self.hidden), "q_proj", dev)
        self.wk = _fp8_bytes(weights[prefix + "k_proj"], (kvd, self.hidden), "k_proj", dev)
        self.wv = _fp8_bytes(weights[prefix + "v_proj"], (kvd, self.hidden), "v_proj", dev)
        self.wo = _fp8_bytes(weights[prefix + "o_proj"], (self.hidden, qd), "o_proj", dev)
        norm = weights.get(prefix + "input_layernorm")
        # nn.RMSNorm's own weight starts at ones (engine.py:85-88)
        self.norm_w = (torch.ones(self.hidden, dtype=torch.float16, device=dev) if norm is None
                       else norm.to(dev, torch.float16).contiguous())
        self._k = self._v = None
        self._len = 0
        self._struct = _lib.Attn(self.n_q, self.n_kv, self.wq.data_ptr(), self.wk.data_ptr(),
                                 self.wv.data_ptr(), self.wo.data_ptr(), self.norm_w.data_ptr())

    # -- the cache ------------------------------------------------------------
    @property
    def capacity(self) -> int:
        return 0 if self._k is None else int(self._k.shape[2])

    def _alloc(self, B: int, cap: int):
        shape = (B, self.n_kv, cap, HEAD_DIM)
        return (torch.empty(shape, dtype=torch.float16, device=self.device),
                torch.empty(shape, dtype=torch.float16, device=self.device))

    @staticmethod
    def _room(need: int) -> int:
        cap = 256
        while cap < need:
            cap *= 2
        return cap

    def rewind(self, n: int) -> None:
        """Roll this layer's cache back to its first n positions, so that a
        call passing views of length n appends in place at position n (a
        rolled-back draft, or one position decoded again).  Unlike every other
        path, this rewrites positions >= n of the buffer: views returned
        earlier that reach past n see those positions change."""
        n = int(n)
        if self._k is None or not 0 <= n <= self._len:
            raise ValueError(f"rewind to {n} positions of a cache holding {self._len}")
        self._len = n

    def _own_view(self, k: torch.Tensor, B: int) -> bool:
        """k is the latest view this layer returned: appending to it in place
        leaves every earlier returned view as it was (they end at or before
        the positions written)."""
        return (self._k is not None and k.is_cuda and k.data_ptr() == self._k.data_ptr()
                and tuple(k.shape[:2]) == (B, self.n_kv) and k.shape[3] == HEAD_DIM
                and k.stride() == self._k.stride() and k.shape[2] == self._len)

    def _prepare_cache(self, B: int, T: int, kv_cache):
        if kv_cache is None:
            # a new sequence gets a new buffer, as the reference's torch.cat
            # returns fresh tensors: views returned for an earlier sequence
            # keep their contents
            self._k, self._v = self._alloc(B, self._room(T))
            return 0
        k_in, v_in = kv_cache
        past = int(k_in.shape[2])
        if tuple(k_in.shape) != (B, self.n_kv, past, HEAD_DIM) or tuple(v_in.shape) != tuple(k_in.shape):
            raise ValueError(f"kv cache of shape {tuple(k_in.shape)} / {tuple(v_in.shape)}, expected "
                             f"({B}, {self.n_kv}, S, {HEAD_DIM})")
        if self._own_view(k_in, B) and v_in.data_ptr() == self._v.data_ptr():
            if past + T > self.capacity:
                k, v = self._alloc(B, self._room(past + T))
                k[:, :, :past].copy_(self._k[:, :, :past])
                v[:, :, :past].copy_(self._v[:, :, :past])
                self._k, self._v = k, v
            return past
        k, v = self._alloc(B, self._room(past + T))
        k[:, :, :past].copy_(k_in)
        v[:, :, :past].copy_(v_in)
        self._k, self._v = k, v
        return past

    # -- forward ---------------------------------------------------------------
    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, kv_cache=None,
                residual_out: torch.Tensor | None = None):
        """x (B, T, H) fp16; cos / sin the engine's tables for the call's
        positions (at least T rows of head_dim / 2); kv_cache None or (k, v).
        Returns (out, (k, v)) as engine.py:90-125.  With ``residual_out``
        (B, T, H) fp16 the kernel also writes x + out there, the engine's
        residual add (engine.py:427)."""
        if x.dtype != torch.float16 or x.dim() != 3 or x.shape[2] != self.hidden:
            raise TypeError(f"x must be (B, T, {self.hidden}) fp16, got {tuple(x.shape)} {x.dtype}")
        B, T, H = x.shape
        if cos.shape[0] < T or sin.shape[0] < T or cos.shape[-1] != HEAD_DIM // 2:
            raise ValueError(f"RoPE tables {tuple(cos.shape)} for {T} positions of head_dim {HEAD_DIM}")
        L = _lib.lib()
        past = self._prepare_cache(B, T, kv_cache)
        xc = x.contiguous()
        c = cos[:T].to(self.device, torch.float32).contiguous()
        s = sin[:T].to(self.device, torch.float32).contiguous()
        out = torch.empty((B, T, H), dtype=torch.float16, device=self.device)
        if residual_out is not None and (residual_out.shape != x.shape or residual_out.dtype != torch.float16
                                         or not residual_out.is_contiguous()):
            raise ValueError("residual_out must be a contiguous fp16 tensor shaped like x")
        cap = self.capacity
        nbytes = L.oi2_attn_workspace_bytes(B, T, self.n_q, self.n_kv, past)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        _lib.check(L.oi2_attn_forward(
            xc.data_ptr(), B, T, ctypes.byref(self._struct), self.eps, c.data_ptr(), s.data_ptr(),
            self._k.data_ptr(), self._v.data_ptr(), cap, past, int(kv_cache is None), out.data_ptr(),
            _lib.ptr(residual_out), ws.data_ptr(), nbytes, _lib.stream_handle(self.device)))
        self._len = past + T
        return out, (self._k[:, :, :past + T], self._v[:, :, :past + T])
