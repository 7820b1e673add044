"""Drop-in hot/cold FFN layer: ``sparse_ffn`` and ``SparseFFNLayer`` with the
reference's call surface (engine.py:163-312), computed by the fused HIP
kernels.

``sparse_ffn`` takes the reference's own dense tensors (fp16 hot, fp32 cold)
and runs them through dense-weight GEMV kernels; the layer below keeps its
weights in compact form.  Differences in representation, not in meaning:
  * hot weights stay fp8 in HBM (``HotWeights``) instead of being widened to
    fp16 at load (engine.py:258-260);
  * the cold "fetch" result is a ``ColdNeurons`` handle - the layer's resident
    INT4 records plus the active slot list on the device - instead of three
    dequantised fp32 tensors (engine.py:266-272); the FFN kernel gathers and
    dequantises the records itself;
  * the predictor's mask never leaves the device: the active list is
    compacted on the GPU (engine.py:274-283 does ``nonzero().tolist()`` and a
    Python filter), so ``submit_cold_fetch`` enqueues work and returns at once.
"""
from __future__ import annotations

import ctypes
from concurrent.futures import Future

import numpy as np
from pathlib import Path
from typing import Optional

import torch

from . import _lib
from .hot import HotWeights
from .store import ColdSection, ColdWeightStore

HIDDEN = _lib.HIDDEN


class ColdNeurons:
    """Active cold neurons of one layer: records + (chunked) slot list."""

    def __init__(self, section: ColdSection | None, slots: torch.Tensor | None,
                 counts: torch.Tensor | None, n_chunks: int, chunk: int, ids=None,
                 gate_bias: torch.Tensor | None = None, expected: int = 0):
        self.expected = expected
        self.section = section
        self.slots = slots
        self.counts = counts
        self.n_chunks = n_chunks
        self.chunk = chunk
        self.ids = ids
        self.gate_bias = gate_bias

    @classmethod
    def from_slots(cls, section: ColdSection | None, slots, gate_bias=None) -> "ColdNeurons":
        """A plain list of record slots (request order)."""
        if section is None:
            return cls(None, None, None, 0, 0)
        dev = section.records.device
        s = torch.as_tensor(slots, dtype=torch.int32).to(dev).reshape(-1)
        n = int(s.shape[0])
        if n == 0:
            return cls(section, None, None, 0, 0)
        counts = torch.tensor([n], dtype=torch.int32, device=dev)
        return cls(section, s, counts, 1, n, gate_bias=gate_bias)

    @classmethod
    def from_ids(cls, section: ColdSection | None, neuron_ids, gate_bias=None) -> "ColdNeurons":
        """read_neurons semantics: request order, absent ids skipped."""
        if section is None:
            return cls(None, None, None, 0, 0)
        return cls.from_slots(section, section.slots_for(neuron_ids), gate_bias)

    def empty(self) -> bool:
        return self.section is None or self.n_chunks == 0

    def structs(self):
        if self.empty():
            return None, None
        return (self.section.struct(self.gate_bias),
                _lib.Active(self.slots.data_ptr(), self.counts.data_ptr(), self.n_chunks,
                            self.chunk, self.expected))

    def capacity(self) -> int:
        return 0 if self.empty() else self.n_chunks * self.chunk

    def count(self) -> int:
        """Number of active records (synchronises with the device)."""
        if self.empty():
            return 0
        return int(self.counts.clamp(0, self.chunk).sum().item())


class _Ready:
    """Completed future: the fetch is already ordered on the device stream."""

    def __init__(self, value):
        self._value = value

    def result(self, timeout=None):
        return self._value

    def done(self):
        return True


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """nn.RMSNorm over the last dim of fp16 x (engine.py:247-249), on the GPU:
    fp16(x * rsqrt(mean(x^2) + eps) * w) - the same arithmetic the FFN and
    predictor kernels apply to their input."""
    shape = x.shape
    x2 = x.reshape(-1, HIDDEN).to(torch.float16).contiguous()
    w = weight.to(device=x2.device, dtype=torch.float16).contiguous()
    out = torch.empty_like(x2)
    _lib.check(_lib.lib().oi2_rmsnorm(x2.data_ptr(), w.data_ptr(), x2.shape[0], ctypes.c_float(eps),
                                      out.data_ptr(), _lib.stream_handle(x2.device)))
    return out.reshape(shape)


def workspace_bytes(batch: int, hot: HotWeights | None, cold: ColdNeurons | None) -> int:
    """Bytes of the scratch buffer oi2_ffn_forward needs for this batch and halves."""
    n_hot = hot.n_hot if hot is not None and hot.n_hot > 0 else 0
    return int(_lib.lib().oi2_ffn_workspace_bytes(batch, n_hot, cold.capacity() if cold is not None else 0))


def _ffn(x2d, norm_w, eps, hot: HotWeights | None, cold: ColdNeurons | None, activation,
         act_on_both, add_residual, out_dtype=torch.float16, want_y32=False, workspace=None,
         xn_in=None, next_norm_w=None, next_eps=None):
    """One oi2_ffn_forward call.  ``workspace`` (uint8 device tensor of at least
    workspace_bytes(...)) is used instead of a fresh allocation when given; its
    contents on entry do not matter.

    With ``xn_in`` or ``next_norm_w`` (batch >= 2) it is one oi2_ffn_forward_chain
    call: ``xn_in`` is RMSNorm(x) as the previous layer's call wrote it (no norm
    launch), and with ``next_norm_w`` the call also returns the next layer's
    normalised rows, (out, xn_next) or (out, y32, xn_next)."""
    dev = x2d.device
    x2d = x2d.to(torch.float16).contiguous()
    B = x2d.shape[0]
    L = _lib.lib()
    hot_s = hot.struct() if hot is not None and hot.n_hot > 0 else None
    cold_s, act_s = cold.structs() if cold is not None else (None, None)
    n_hot = hot.n_hot if hot_s is not None else 0
    ws_bytes = L.oi2_ffn_workspace_bytes(B, n_hot, cold.capacity() if cold is not None else 0)
    if workspace is not None:
        if workspace.dtype != torch.uint8 or workspace.device != dev or workspace.numel() < ws_bytes:
            raise ValueError(f"workspace must be a uint8 tensor of >= {ws_bytes} bytes on {dev}")
        ws = workspace
    else:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty_like(x2d)
    y32 = torch.empty((B, HIDDEN), dtype=torch.float32, device=dev) if want_y32 else None
    act = _lib.ACT_RELU if activation == "relu" else _lib.ACT_SILU
    hot_p = ctypes.byref(hot_s) if hot_s is not None else None
    cold_p = ctypes.byref(cold_s) if cold_s is not None else None
    act_p = ctypes.byref(act_s) if act_s is not None else None
    if xn_in is None and next_norm_w is None:
        _lib.check(L.oi2_ffn_forward(
            x2d.data_ptr(), B, _lib.ptr(norm_w), ctypes.c_float(eps), hot_p, cold_p, act_p,
            act, int(bool(act_on_both)), int(bool(add_residual)), out.data_ptr(), _lib.ptr(y32),
            ws.data_ptr(), ws_bytes, _lib.stream_handle(dev)))
        return (out, y32) if want_y32 else out
    if xn_in is not None and (xn_in.dtype != torch.float16 or tuple(xn_in.shape) != tuple(x2d.shape)
                              or not xn_in.is_contiguous()):
        raise ValueError(f"xn_in must be a contiguous fp16 tensor of shape {tuple(x2d.shape)}")
    xn_next = torch.empty_like(x2d) if next_norm_w is not None else None
    _lib.check(L.oi2_ffn_forward_chain(
        x2d.data_ptr(), B, _lib.ptr(norm_w), ctypes.c_float(eps), _lib.ptr(xn_in), hot_p, cold_p, act_p,
        act, int(bool(act_on_both)), int(bool(add_residual)), out.data_ptr(), _lib.ptr(y32),
        _lib.ptr(next_norm_w), ctypes.c_float(eps if next_eps is None else next_eps), _lib.ptr(xn_next),
        ws.data_ptr(), ws_bytes, _lib.stream_handle(dev)))
    res = (out, y32) if want_y32 else (out,)
    return res + (xn_next,) if next_norm_w is not None else (res if want_y32 else out)


_DENSE_DTYPES = (torch.float16, torch.float32, torch.bfloat16)


def _dense_half(gate, up, down, what):
    """Validate one half given as the reference's tensors: gate/up (n, H),
    down (H, n), one float dtype; returns (n, dtype code, g, u, d) with the
    tensors contiguous, or (0, ...) for an absent or empty half
    (engine.py:194, :199: a half is used when gate.shape[0] > 0)."""
    if gate is None or gate.shape[0] == 0:
        return 0, _lib.DTYPE_F16, None, None, None
    if up is None or down is None:
        raise TypeError(f"{what}: gate, up and down must all be given")
    n = int(gate.shape[0])
    if tuple(gate.shape) != (n, HIDDEN) or tuple(up.shape) != (n, HIDDEN) or \
            tuple(down.shape) != (HIDDEN, n):
        raise ValueError(f"{what}: gate/up must be ({n}, {HIDDEN}) and down ({HIDDEN}, {n}); got "
                         f"{tuple(gate.shape)}, {tuple(up.shape)}, {tuple(down.shape)}")
    if gate.dtype not in _DENSE_DTYPES or up.dtype != gate.dtype or down.dtype != gate.dtype:
        raise TypeError(f"{what}: weights must share one of fp16 / fp32 / bf16, got "
                        f"{gate.dtype}, {up.dtype}, {down.dtype}")
    return n, _lib.dtype_code(gate.dtype), gate.contiguous(), up.contiguous(), down.contiguous()


def _sparse_ffn_dense(x2d, activation, act_on_both, hot, cold):
    """oi2_sparse_ffn_dense: both halves as dense tensors; fp32 y."""
    dev = x2d.device
    n_hot, hdt, gh, uh, dh = hot
    n_cold, cdt, gc, uc, dc = cold
    B = x2d.shape[0]
    L = _lib.lib()
    ws_bytes = L.oi2_sparse_ffn_dense_workspace_bytes(B, n_hot, n_cold)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    y32 = torch.empty((B, HIDDEN), dtype=torch.float32, device=dev)
    act = _lib.ACT_RELU if activation == "relu" else _lib.ACT_SILU
    _lib.check(L.oi2_sparse_ffn_dense(
        x2d.data_ptr(), B, act, int(bool(act_on_both)), n_hot, hdt, _lib.ptr(gh), _lib.ptr(uh),
        _lib.ptr(dh), n_cold, cdt, _lib.ptr(gc), _lib.ptr(uc), _lib.ptr(dc), None, y32.data_ptr(),
        ws.data_ptr(), ws_bytes, _lib.stream_handle(dev)))
    return y32


def sparse_ffn(x: torch.Tensor, activation: str, act_on_both: bool,
               gate_hot=None, up_hot=None, down_hot=None,
               gate_cold=None, up_cold=None, down_cold=None):
    """engine.py:173-209: hot half + cold half of the gated FFN for x (B, H)
    fp16, returned in x.dtype.

    Each half comes in either of two forms:
      * the reference's own tensors (what SparseFFNLayer and read_neurons
        hand it): gate/up (n, H), down (H, n), fp16 (the widened hot file),
        fp32 (dequantised cold records) or bf16 - computed by the dense-weight
        HIP GEMV kernels (oi2_sparse_ffn_dense);
      * this library's compact handles: the whole hot half as one HotWeights
        in ``gate_hot`` (fp8 in HBM) and the whole cold half as one
        ColdNeurons in ``gate_cold`` (INT4 records + active list), with the
        up/down arguments None - computed by the fused fp8 / INT4 kernels.
    Either half may be None or empty; both empty gives zeros (:207-208).
    Accumulation is fp32 throughout; the halves are summed in fp32 and
    rounded once to x.dtype.  The kernels read fp16 activations (the
    engine's); a bf16 or fp32 x is rounded to fp16 first (exact for bf16
    values in fp16's range)."""
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise TypeError(f"x must be floating point (fp16, bf16 or fp32), got {x.dtype}")
    x2d = x.reshape(-1, HIDDEN).to(torch.float16).contiguous()
    hot_handle = isinstance(gate_hot, HotWeights)
    cold_handle = isinstance(gate_cold, ColdNeurons)
    if hot_handle and (up_hot is not None or down_hot is not None):
        raise TypeError("with a HotWeights in gate_hot, up_hot and down_hot must be None")
    if cold_handle and (up_cold is not None or down_cold is not None):
        raise TypeError("with a ColdNeurons in gate_cold, up_cold and down_cold must be None")
    for t, what in ((gate_hot, "gate_hot"), (gate_cold, "gate_cold")):
        if t is not None and not isinstance(t, (HotWeights, ColdNeurons, torch.Tensor)):
            raise TypeError(f"{what}: expected a tensor or a library handle, got {type(t).__name__}")
    hot_dense = None if hot_handle else _dense_half(gate_hot, up_hot, down_hot, "hot half")
    cold_dense = None if cold_handle else _dense_half(gate_cold, up_cold, down_cold, "cold half")
    y = None
    if hot_dense is not None or cold_dense is not None:
        none = (0, _lib.DTYPE_F16, None, None, None)
        y = _sparse_ffn_dense(x2d, activation, act_on_both, hot_dense or none, cold_dense or none)
    if hot_handle or cold_handle:
        _, y2 = _ffn(x2d, None, 0.0, gate_hot if hot_handle else None,
                     gate_cold if cold_handle else None, activation, act_on_both,
                     add_residual=False, want_y32=True)
        y = y2 if y is None else y + y2
    return y.to(x.dtype).reshape(x.shape)


class SparseFFNLayer(torch.nn.Module):
    """engine.py:212-312 with the same constructor and methods."""

    _EID = 0

    def __init__(self, layer_idx: int, hot_dir: str, cold_store: ColdWeightStore,
                 predictor, cfg: dict, device, executor=None, ffn_norm_weight=None,
                 threshold: float = 0.5, hot: HotWeights | None = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.cold_store = cold_store
        self.predictor = predictor
        self.device = torch.device(device)
        self.executor = executor
        self.activation = cfg.get("hidden_act", "silu")
        self.act_on_both = cfg.get("act_on_both", False)
        self.inter_dim = cfg["intermediate_dim"]
        self.eps = float(cfg["rms_norm_eps"])
        self.threshold = threshold
        H = cfg["hidden_dim"]
        if H != HIDDEN:
            raise ValueError(f"hidden_dim {H}: the kernels are built for {HIDDEN}")
        w = ffn_norm_weight if ffn_norm_weight is not None else torch.ones(H)
        self.norm_weight = w.to(device=self.device, dtype=torch.float16).contiguous()
        self.hot = hot
        if self.hot is None:
            p = Path(hot_dir) / f"layer_{layer_idx:03d}_expert_{self._EID:03d}.pt"
            if p.exists():
                self.hot = HotWeights.load(str(p), self.device)
        self._hot_id_set = set(self.hot.neuron_ids.tolist()) if self.hot is not None else set()
        self._section = cold_store.section(layer_idx, self._EID) if cold_store is not None else None
        self._n_chunks = (self.inter_dim + _lib.SEL_CHUNK - 1) // _lib.SEL_CHUNK
        self._lut = self._section.lut if self._section is not None else None
        # file residency: each fetch reads the records from the file on the
        # executor (engine.py:266-272), copies them to the device on a copy
        # stream, and hands the FFN a section over the copy
        self._file = (cold_store is not None and getattr(cold_store, "residency", "hbm") == "file"
                      and self._section is not None)
        if self._file:
            self._copy_stream = torch.cuda.Stream(device=self.device)
            self._arange = torch.arange(max(self._section.n_records, 1), dtype=torch.int32,
                                        device=self.device)
            self._inflight = []          # (copy event, pinned buffer) until the copy has run

    # ── cold selection ──
    def _cold_ids_for(self, x_normed: torch.Tensor) -> list[int]:
        """engine.py:274-283 as a host list (debug / compatibility helper; the
        forward path keeps the list on the device)."""
        sel = self._select(x_normed, normed=True)
        if sel.empty():
            return []
        ids = []
        counts = sel.counts.cpu().tolist()
        cpu_ids = sel.ids.cpu()
        for c, n in enumerate(counts):
            ids.extend(cpu_ids[c * sel.chunk: c * sel.chunk + n].tolist())
        return ids

    def _select(self, x: torch.Tensor, normed: bool) -> ColdNeurons:
        sec = self._section
        if sec is None:
            return ColdNeurons(None, None, None, 0, 0)
        pred = None
        if self.predictor is not None:
            pred = (self.predictor.get(self.layer_idx, self._EID)
                    if hasattr(self.predictor, "get") else self.predictor)
        if pred is None:
            # no predictor: every cold neuron, ascending id order
            slots = sec.all_slots()
            return ColdNeurons(sec, slots, torch.tensor([slots.shape[0]], dtype=torch.int32,
                                                        device=self.device),
                               1, max(1, int(slots.shape[0])))
        q = x[:, -1, :] if x.dim() == 3 else x.reshape(-1, HIDDEN)
        q = q.to(torch.float16).contiguous()
        nc = self._n_chunks
        dev = self.device
        slots = torch.empty(nc * _lib.SEL_CHUNK, dtype=torch.int32, device=dev)
        ids = torch.empty(nc * _lib.SEL_CHUNK, dtype=torch.int32, device=dev)
        counts = torch.empty(nc, dtype=torch.int32, device=dev)
        p = pred.struct()
        L = _lib.lib()
        ws_bytes = L.oi2_predict_workspace_bytes(ctypes.byref(p))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(L.oi2_predict_select(
            q.data_ptr(), q.shape[0], None if normed else self.norm_weight.data_ptr(),
            ctypes.c_float(self.eps), ctypes.byref(p), _lib.logit_threshold(self.threshold),
            sec.lut.data_ptr(), slots.data_ptr(), ids.data_ptr(), counts.data_ptr(), None, None,
            None, ws.data_ptr(), ws_bytes, _lib.stream_handle(dev)))
        return ColdNeurons(sec, slots, counts, nc, _lib.SEL_CHUNK, ids=ids)

    def _cold_slots_host(self, x: torch.Tensor, normed: bool) -> np.ndarray:
        """The record slots of _cold_ids_for's list, ascending neuron id, on
        the host (the list the reference hands its executor, engine.py:289)."""
        sel = self._select(x, normed)
        if sel.empty():
            return np.zeros(0, np.int32)
        counts = sel.counts.cpu().tolist()
        slots = sel.slots.cpu().numpy()
        parts = [slots[c * sel.chunk: c * sel.chunk + min(max(n, 0), sel.chunk)]
                 for c, n in enumerate(counts)]
        return np.concatenate(parts).astype(np.int32) if parts else np.zeros(0, np.int32)

    def _fetch_file(self, slots: np.ndarray) -> ColdNeurons:
        """engine.py:266-272 (_fetch_cold) with file residency: read the
        records from the file into pinned memory and copy them to the device
        on the copy stream; the result carries the copy's event."""
        n = int(slots.shape[0])
        if n == 0:
            return ColdNeurons(None, None, None, 0, 0)
        cs = self._copy_stream
        with torch.cuda.stream(cs):
            counts = torch.full((1,), n, dtype=torch.int32, device=self.device)
            staged = self.cold_store.fetch_records(self._section, slots, cs)
        cold = ColdNeurons(staged, self._arange[:n], counts, 1, n)
        cold.event = staged.event
        return cold

    def submit_cold_fetch(self, x: torch.Tensor):
        """engine.py:285-290: predict this layer's cold set from x (normalised
        with this layer's norm) and return an object with ``.result()``.  With
        a device-resident store the work is only enqueued on the stream, so
        the returned future is already complete; with file residency the
        fetch runs on the executor (inline without one)."""
        with torch.no_grad():
            if not self._file:
                return _Ready(self._select(x, normed=False))
            slots = self._cold_slots_host(x, normed=False)
            if self.executor is not None:
                return self.executor.submit(self._fetch_file, slots)
            return _Ready(self._fetch_file(slots))

    def forward(self, x: torch.Tensor, prefetch_future=None) -> torch.Tensor:
        """engine.py:292-312: residual + FFN(RMSNorm(x)) for x (B, T, H)."""
        B, T, H = x.shape
        if prefetch_future is not None:
            cold = prefetch_future.result()
        elif self._file:
            cold = self._fetch_file(self._cold_slots_host(x, normed=False))
        else:
            cold = self._select(x, normed=False)
        if isinstance(cold, Future):
            cold = cold.result()
        stream = torch.cuda.current_stream(self.device)
        ev = getattr(cold, "event", None)
        if ev is not None:
            stream.wait_event(ev)
        out = _ffn(x.reshape(B * T, H), self.norm_weight, self.eps, self.hot, cold,
                   self.activation, self.act_on_both, add_residual=True)
        if ev is not None:
            # the staged records are read on this stream; their pinned buffer
            # is released once the copy has run
            cold.section.records.record_stream(stream)
            self._inflight = [(e, h) for e, h in self._inflight if not e.query()]
            self._inflight.append((ev, cold.section.host_buffer))
        return out.reshape(B, T, H).to(x.dtype)
