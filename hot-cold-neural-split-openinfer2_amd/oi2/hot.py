"""Hot FP8 neurons of one layer, resident in device memory.

File format (splitter.py:221-226): ``hot_weights/layer_{L:03d}_expert_000.pt`` =
{"neuron_ids": int64 ascending, "gate": (n_hot, H) fp8, "up": (n_hot, H) fp8,
"down": (H, n_hot) fp8}.  The reference widens these to fp16 at load
(engine.py:258-260); here they stay fp8 in HBM, with optional per-row fp32
scales under "gate_scale" / "up_scale" / "down_scale" (absent = 1.0, which is
the reference's unscaled cast).  The down matrix is stored with its rows padded
to a multiple of 64 bytes so every row starts 16-byte aligned.
"""
from __future__ import annotations

import os

import torch

from . import _lib

HIDDEN = _lib.HIDDEN
FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


def _pad_stride(n: int) -> int:
    return max(64, (n + 63) // 64 * 64)


def quantize_fp8_rows(w: torch.Tensor, per_row_scale: bool = True):
    """fp32 rows -> (fp8 codes as uint8, fp32 scale per row).  With a scale,
    s = max|row| / 448 and codes = fp8(row / s) (torch's RNE cast); without,
    s = 1 and codes = fp8(row) as splitter.py:223-225 writes them."""
    w = w.float()
    if per_row_scale:
        s = w.abs().amax(dim=1).clamp(min=1e-30) / FP8_MAX
        q = (w / s[:, None]).to(FP8)
    else:
        s = torch.ones(w.shape[0], dtype=torch.float32, device=w.device)
        q = w.to(FP8)
    return q.view(torch.uint8), s.float()


class HotWeights:
    """Device-resident hot half: gate/up (n_hot, H), down (H, stride)."""

    def __init__(self, neuron_ids, gate_q, up_q, down_q, gate_scale, up_scale, down_scale,
                 gate_bias=None):
        n = int(gate_q.shape[0])
        self.n_hot = n
        self.neuron_ids = neuron_ids.to(torch.int64)
        dev = gate_q.device
        self.device = dev
        self.gate_q = gate_q.contiguous()
        self.up_q = up_q.contiguous()
        stride = _pad_stride(n)
        self.down_stride = stride
        dq = torch.zeros((HIDDEN, stride), dtype=torch.uint8, device=dev)
        dq[:, :n] = down_q
        self.down_q = dq
        self.gate_scale = gate_scale.float().contiguous()
        self.up_scale = up_scale.float().contiguous()
        self.down_scale = down_scale.float().contiguous()
        self.gate_bias = None if gate_bias is None else gate_bias.float().contiguous()
        if self.gate_q.shape != (n, HIDDEN) or self.up_q.shape != (n, HIDDEN):
            raise ValueError("hot gate/up must be (n_hot, 4096)")
        if down_q.shape != (HIDDEN, n):
            raise ValueError("hot down must be (4096, n_hot)")

    # ── constructors ──
    @classmethod
    def from_dense(cls, neuron_ids, gate, up, down, per_row_scale=True, gate_bias=None):
        """gate/up (n, H), down (H, n) float tensors on the target device."""
        gq, gs = quantize_fp8_rows(gate, per_row_scale)
        uq, us = quantize_fp8_rows(up, per_row_scale)
        dq, ds = quantize_fp8_rows(down, per_row_scale)
        return cls(torch.as_tensor(neuron_ids), gq, uq, dq, gs, us, ds, gate_bias)

    @classmethod
    def load(cls, path: str, device) -> "HotWeights":
        """Load a split hot file; tensors are read without unpickling code."""
        w = torch.load(path, map_location="cpu", weights_only=True)
        dev = torch.device(device)

        def codes(t):
            if t.dtype == FP8:
                return t.view(torch.uint8).to(dev)
            if t.dtype == torch.uint8:
                return t.to(dev)
            raise ValueError(f"hot tensor dtype {t.dtype} is not fp8")
        g, u, d = codes(w["gate"]), codes(w["up"]), codes(w["down"])
        n = g.shape[0]
        ones_n = torch.ones(n, dtype=torch.float32, device=dev)
        ones_h = torch.ones(HIDDEN, dtype=torch.float32, device=dev)
        return cls(w["neuron_ids"], g, u, d,
                   w.get("gate_scale", ones_n).to(dev), w.get("up_scale", ones_n).to(dev),
                   w.get("down_scale", ones_h).to(dev), w.get("gate_bias"))

    def save(self, path: str):
        """Write in the split layout (fp8 tensors) plus the scale keys."""
        n = self.n_hot
        torch.save({
            "neuron_ids": self.neuron_ids.cpu(),
            "gate": self.gate_q.cpu().view(FP8),
            "up": self.up_q.cpu().view(FP8),
            "down": self.down_q[:, :n].cpu().contiguous().view(FP8),
            "gate_scale": self.gate_scale.cpu(),
            "up_scale": self.up_scale.cpu(),
            "down_scale": self.down_scale.cpu(),
        }, path)

    def struct(self) -> _lib.Hot:
        return _lib.Hot(self.n_hot, self.down_stride, self.gate_q.data_ptr(), self.up_q.data_ptr(),
                        self.down_q.data_ptr(), self.gate_scale.data_ptr(),
                        self.up_scale.data_ptr(), self.down_scale.data_ptr(),
                        _lib.ptr(self.gate_bias))

    def nbytes(self) -> int:
        return 3 * self.n_hot * HIDDEN

    @staticmethod
    def path_for(hot_dir: str, layer_idx: int, expert_idx: int = 0) -> str:
        return os.path.join(hot_dir, f"layer_{layer_idx:03d}_expert_{expert_idx:03d}.pt")
