"""Low-rank activation predictor on the GPU: NeuronPredictor and
PredictorRegistry with the reference's interface (predictor.py:55-96,
413-462), evaluated by the predictor kernels.

Weights keep the file's dtype (fp32 as trained, or bf16) unless a dtype is
asked for at load; the hidden state, of whatever float dtype the caller holds
it in, is cast straight to that dtype first (predictor.py:455).  The mask is sigmoid(logit) >=
threshold, decided in logit space (logit >= log(p / (1 - p))), which is the same
set except for logits within float rounding of the threshold.
"""
from __future__ import annotations

import os
from pathlib import Path

import torch

from . import _lib

HIDDEN = _lib.HIDDEN


class NeuronPredictor:
    """sigmoid(up(down(x))): down = (rank, H) no bias, up = (I, rank) + bias
    (predictor.py:67-68)."""

    def __init__(self, down_w: torch.Tensor, up_w: torch.Tensor, up_b: torch.Tensor):
        if down_w.dtype != up_w.dtype or down_w.dtype != up_b.dtype:
            raise ValueError("predictor weights must share one dtype")
        if down_w.dtype not in (torch.float32, torch.bfloat16):
            raise ValueError(f"predictor dtype {down_w.dtype} (fp32 or bf16 supported)")
        self.rank, self.hidden_dim = down_w.shape
        self.intermediate_dim = up_w.shape[0]
        if self.hidden_dim != HIDDEN or up_w.shape[1] != self.rank or up_b.shape != (self.intermediate_dim,):
            raise ValueError("predictor shapes must be (rank, 4096), (I, rank), (I,)")
        self.down_w = down_w.contiguous()
        self.up_w = up_w.contiguous()
        self.up_b = up_b.contiguous()
        self.dtype = down_w.dtype
        self.device = down_w.device

    @classmethod
    def load(cls, path: str, device="cuda", dtype=torch.float32) -> "NeuronPredictor":
        """predictor.py:83-96 file layout: {"hidden_dim", "intermediate_dim",
        "rank", "state_dict": {"down.weight", "up.weight", "up.bias"}}.  The
        reference loads the state dict into a freshly built (float32) module,
        so its parameters are float32 whatever the file holds; ``dtype`` keeps
        that default (None keeps the file's own dtype, torch.bfloat16 halves
        the predictor's bytes)."""
        ckpt = torch.load(path, map_location="cpu", weights_only=True)
        sd = ckpt["state_dict"]
        t = [sd["down.weight"], sd["up.weight"], sd["up.bias"]]
        if dtype is not None:
            t = [v.to(dtype) for v in t]
        return cls(*(v.to(device) for v in t))

    def save(self, path: str):
        torch.save({"hidden_dim": self.hidden_dim, "intermediate_dim": self.intermediate_dim,
                    "rank": self.rank,
                    "state_dict": {"down.weight": self.down_w.cpu(), "up.weight": self.up_w.cpu(),
                                   "up.bias": self.up_b.cpu()}}, path)

    def struct(self) -> _lib.Predictor:
        return _lib.Predictor(self.intermediate_dim, self.rank,
                              _lib.DTYPE_BF16 if self.dtype == torch.bfloat16 else _lib.DTYPE_F32,
                              self.down_w.data_ptr(), self.up_w.data_ptr(), self.up_b.data_ptr())

    def _run(self, x: torch.Tensor, threshold: float, want_probs: bool, want_mask: bool,
             want_logits: bool = False):
        lead = x.shape[:-1]
        h = x.reshape(-1, HIDDEN).to(device=self.device)
        if h.dtype not in (torch.float16, torch.float32, torch.bfloat16):
            h = h.float()
        h = h.contiguous()
        rows = h.shape[0]
        I = self.intermediate_dim
        logits = torch.empty((rows, I), dtype=torch.float32, device=self.device) if want_logits else None
        probs = torch.empty((rows, I), dtype=torch.float32, device=self.device) if want_probs else None
        mask = torch.empty((rows, I), dtype=torch.bool, device=self.device) if want_mask else None
        p = self.struct()
        L = _lib.lib()
        ws_bytes = L.oi2_predict_workspace_bytes(ctypes_ref(p))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=self.device)
        _lib.check(L.oi2_predict(h.data_ptr(), _lib.dtype_code(h.dtype), rows, ctypes_ref(p),
                                 _lib.logit_threshold(threshold),
                                 _lib.ptr(logits), _lib.ptr(probs), _lib.ptr(mask), ws.data_ptr(),
                                 ws_bytes, _lib.stream_handle(self.device)))
        out = []
        for t in (logits, probs, mask):
            if t is not None:
                out.append(t.reshape(*lead, I))
        return out[0] if len(out) == 1 else tuple(out)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """Probabilities (..., I) fp32.  x (fp16, fp32 or bf16; other float
        dtypes go through fp32) is cast straight to the predictor's dtype, as
        PredictorRegistry.predict does (predictor.py:455)."""
        return self._run(x, 0.5, want_probs=True, want_mask=False)

    __call__ = forward

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        return self._run(x, 0.5, want_probs=False, want_mask=False, want_logits=True)

    def predict_mask(self, x: torch.Tensor, threshold: float = 0.5) -> torch.Tensor:
        """predictor.py:77-79: bool (..., I)."""
        return self._run(x, threshold, want_probs=False, want_mask=True)


def ctypes_ref(s):
    import ctypes
    return ctypes.byref(s)


class PredictorRegistry:
    """predictor.py:413-462: every ``layer_*_expert_*.pt`` in a directory,
    resident on the device, looked up by (layer, expert)."""

    def __init__(self, predictor_dir: str, device="cuda", dtype=torch.float32):
        self.predictors: dict[tuple[int, int], NeuronPredictor] = {}
        self.device = device
        for f in sorted(Path(predictor_dir).glob("layer_*_expert_*.pt")):
            parts = f.stem.split("_")
            self.predictors[(int(parts[1]), int(parts[3]))] = NeuronPredictor.load(
                str(f), device, dtype)

    def get(self, layer_idx: int, expert_idx: int = 0) -> NeuronPredictor | None:
        return self.predictors.get((layer_idx, expert_idx))

    def predict(self, layer_idx: int, expert_idx: int, hidden_state: torch.Tensor,
                threshold: float = 0.5):
        """Bool mask (batch, I) of predicted-active neurons, or None when the
        layer has no predictor (predictor.py:447-449)."""
        p = self.predictors.get((layer_idx, expert_idx))
        if p is None:
            return None
        if hidden_state.dim() == 1:
            hidden_state = hidden_state[None]
        return p.predict_mask(hidden_state, threshold)

    def vram_usage_mb(self) -> float:
        return sum(sum(t.numel() * t.element_size() for t in (p.down_w, p.up_w, p.up_b))
                   for p in self.predictors.values()) / 1e6

    @staticmethod
    def path_for(predictor_dir: str, layer_idx: int, expert_idx: int = 0) -> str:
        return os.path.join(predictor_dir, f"layer_{layer_idx:03d}_expert_{expert_idx:03d}.pt")
