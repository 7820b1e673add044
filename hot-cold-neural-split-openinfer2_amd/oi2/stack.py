"""FFN-only decode stack on the device (the layer loop of engine.py:421-438
without attention), batch 1, one C call per token."""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from .hot import HotWeights
from .predictor import NeuronPredictor

HIDDEN = _lib.HIDDEN


@dataclass
class StackLayer:
    hot: Optional[HotWeights]
    records: Optional[torch.Tensor]       # (n, 6400) uint8 device
    lut: Optional[torch.Tensor]           # (inter,) int32 device
    norm_w: torch.Tensor                  # (H,) fp16 device
    predictor: Optional[NeuronPredictor]
    cold_gate_bias: Optional[torch.Tensor] = None


class DecodeStack:
    def __init__(self, layers: list[StackLayer], inter: int, eps: float, activation: str = "silu",
                 act_on_both: bool = False, threshold_logit: float = 0.0, use_graph: bool = True,
                 staging: int = 0):
        self.layers = layers
        self.inter = inter
        self.n_layers = len(layers)
        self.n_chunks = (inter + _lib.SEL_CHUNK - 1) // _lib.SEL_CHUNK
        arr = (_lib.Layer * self.n_layers)()
        for i, l in enumerate(layers):
            hot = l.hot.struct() if l.hot is not None else _lib.Hot()
            n_rec = int(l.records.shape[0]) if l.records is not None else 0
            cold = _lib.Cold(_lib.ptr(l.records) if n_rec else None, n_rec, _lib.ptr(l.cold_gate_bias))
            pred = l.predictor.struct() if l.predictor is not None else _lib.Predictor()
            arr[i] = _lib.Layer(hot, cold, _lib.ptr(l.lut), l.norm_w.data_ptr(), pred)
        self._arr = arr
        L = _lib.lib()
        h = ctypes.c_void_p()
        act = _lib.ACT_RELU if activation == "relu" else _lib.ACT_SILU
        _lib.check(L.oi2_stack_create(arr, self.n_layers, inter, ctypes.c_float(eps), act,
                                      int(bool(act_on_both)), ctypes.c_float(threshold_logit),
                                      ctypes.byref(h)))
        self._h = h
        _lib.check(L.oi2_stack_set_graph(h, int(bool(use_graph))))
        if staging:
            self.set_staging(staging)

    def set_staging(self, copy_workgroups: int):
        """Copy each layer's active records one layer ahead on a side stream
        into HBM staging buffers, with a copy kernel of `copy_workgroups`
        workgroups (records may then live in pinned host memory); 0: the FFN
        reads the records where they are."""
        _lib.check(_lib.lib().oi2_stack_set_staging(self._h, int(copy_workgroups)))

    def set_token_kernel(self, enable: bool):
        """Run each token as one persistent kernel (the default where the
        configuration allows it) or as two launches per layer."""
        _lib.check(_lib.lib().oi2_stack_set_token_kernel(self._h, int(bool(enable))))

    @property
    def token_kernel(self) -> bool:
        return bool(_lib.lib().oi2_stack_token_kernel(self._h))

    def status(self, stream=None):
        """Wait for the stream; raise OI2Error if a device-side wait (of the
        persistent kernel, or of the staged path) ran past its bound in any
        token decoded since the previous call."""
        dev = self.layers[0].norm_w.device
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(dev)
        _lib.check(_lib.lib().oi2_stack_status(self._h, s or None))

    def set_wait_bound(self, polls: int):
        """Bound, in polls, of the device-side waits of the persistent kernel
        and of the staged path (default 1 << 20).  Past it a wait gives up and
        the next status() raises; meant for tests of that path."""
        _lib.check(_lib.lib().oi2_stack_set_wait_bound(self._h, int(polls)))

    def profile_token(self, x_in: torch.Tensor, x_out: torch.Tensor, stream=None, reps: int = 16):
        """Mean microseconds of the persistent token kernel alone."""
        us = ctypes.c_float()
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_profile_token(self._h, x_in.data_ptr(), x_out.data_ptr(),
                                                      int(reps), ctypes.byref(us), s or None))
        return us.value

    TRACE_POINTS = ("U start", "B1 U inputs in", "B2 U products in", "U arrival issued",
                    "U signal seen", "D1a D inputs in", "D1b next list in", "D arrival issued")

    def trace_token(self, x_in: torch.Tensor, x_out: torch.Tensor, stream=None) -> torch.Tensor:
        """Decode x_in once on the persistent token kernel with its control
        waves stamping eight points of every layer (TRACE_POINTS) on the
        device's 100 MHz counter.  Returns an int64 device tensor (layers up
        to 64, 256 groups, 8 points) of raw counter values."""
        n = min(len(self.layers), 64)
        t = torch.zeros((n, 256, len(self.TRACE_POINTS)), dtype=torch.int64, device=x_in.device)
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_trace_token(self._h, x_in.data_ptr(), x_out.data_ptr(), t.data_ptr(),
                                                    t.numel() * 8, s or None))
        return t

    def selection_layout(self) -> tuple[int, int]:
        """(n_chunks, chunk) of the active sets trace() returns."""
        nc, ch = ctypes.c_int32(), ctypes.c_int32()
        _lib.check(_lib.lib().oi2_stack_selection_layout(self._h, ctypes.byref(nc), ctypes.byref(ch)))
        return nc.value, ch.value

    def set_expected_active(self, n: int):
        """Size the cold pass for about n active records per layer."""
        _lib.check(_lib.lib().oi2_stack_set_expected_active(self._h, int(n)))

    def decode(self, x_in: torch.Tensor, x_out: torch.Tensor, stream=None):
        """x_out (H) fp16 = the token after every FFN layer."""
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_decode(self._h, x_in.data_ptr(), x_out.data_ptr(), s or None))

    def predict(self, layer: int, x: torch.Tensor, stream=None):
        """Layer `layer`'s cold set predicted from x (H) fp16 (the engine
        predicts layer 0's from the embedded token, engine.py:422)."""
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x.device)
        _lib.check(_lib.lib().oi2_stack_predict(self._h, int(layer), x.data_ptr(), s or None))

    def layer(self, layer: int, x_in: torch.Tensor, x_out: torch.Tensor, stream=None):
        """One layer on its own: x_out = x_in + FFN(RMSNorm(x_in)) over the
        set held for `layer`, and the next layer's set predicted from x_in
        (the engine's lookahead from the post-attention state,
        engine.py:431-436).  For callers that run attention between layers."""
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_layer(self._h, int(layer), x_in.data_ptr(), x_out.data_ptr(), s or None))

    def profile(self, x_in: torch.Tensor, x_out: torch.Tensor, stream=None, reps: int = 8):
        """Mean (ffn_up us, ffn_down us) per launch: every layer's kernel
        launched back to back `reps` times between two hipEvents on the launch
        stream.  Leaves the stack in the state of decoding x_in."""
        up, down = ctypes.c_float(), ctypes.c_float()
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_profile(self._h, x_in.data_ptr(), x_out.data_ptr(), int(reps),
                                                ctypes.byref(up), ctypes.byref(down), s or None))
        return up.value, down.value

    def profile_staging(self, x_in: torch.Tensor, x_out: torch.Tensor, stream=None, reps: int = 4):
        """Mean microseconds of one layer's record copy (staging enabled)."""
        us = ctypes.c_float()
        s = stream.cuda_stream if stream is not None else _lib.stream_handle(x_in.device)
        _lib.check(_lib.lib().oi2_stack_profile_staging(self._h, x_in.data_ptr(), x_out.data_ptr(),
                                                        int(reps), ctypes.byref(us), s or None))
        return us.value

    def trace(self):
        """(xs (n_layers, H) fp16 layer outputs, counts (n_layers, n_chunks),
        slots, ids (n_layers, n_chunks * chunk)) of the last decode, in the
        chunking selection_layout() reports."""
        dev = self.layers[0].norm_w.device
        n = self.n_layers
        nc, ch = self.selection_layout()
        xs = torch.empty((n, HIDDEN), dtype=torch.float16, device=dev)
        counts = torch.empty((n, nc), dtype=torch.int32, device=dev)
        slots = torch.empty((n, nc * ch), dtype=torch.int32, device=dev)
        ids = torch.empty((n, nc * ch), dtype=torch.int32, device=dev)
        _lib.check(_lib.lib().oi2_stack_trace(self._h, xs.data_ptr(), counts.data_ptr(),
                                              slots.data_ptr(), ids.data_ptr(),
                                              _lib.stream_handle(dev)))
        return xs, counts, slots, ids

    def active_ids(self, layer: int, counts=None, ids=None) -> list[int]:
        """Layer `layer`'s active cold ids of the last decode, ascending."""
        if counts is None:
            _, counts, _, ids = self.trace()
        _, ch = self.selection_layout()
        c = counts[layer].cpu().tolist()
        row = ids[layer].cpu()
        out = []
        for k, m in enumerate(c):
            out.extend(row[k * ch: k * ch + m].tolist())
        return out

    def close(self):
        if self._h:
            _lib.lib().oi2_stack_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
