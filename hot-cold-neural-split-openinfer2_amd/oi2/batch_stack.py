"""FFN-only decode of a batch of tokens with the cold records read from the
split file on every step: DesdemonaEngine.forward's layer loop
(engine.py:406-442) over SparseFFNLayer, for B tokens that share one cold
set per layer, selected from the batch-mean query (engine.py:274-283).

Per layer L the device runs the selection of layer L+1 (predictor on the
batch mean of RMSNorm_{L+1}(x_L), threshold, hot filter, ascending
compaction; engine.py:432-436) ahead of FFN(L).  The host takes the list
back, and a worker thread reads those records from the file (liboi2's native
file store: a mapping of the file, or O_DIRECT page reads) into one of two
pinned buffers, in list order, while the device computes FFN(L) - the
reference's executor-backed prefetch (engine.py:266-272, 285-290).  The same
worker then enqueues one hipMemcpyAsync of them into one of two device
buffers on a copy stream, and FFN(L+1) (the matrix-core batch kernels, B
tokens at once) waits for that copy on the device and reads the records
there through a slot-less list.  A pinned buffer is refilled only after the
copy that last read it has run.
"""
from __future__ import annotations

import ctypes
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _lib
from . import format as fmt
from .filestore import FileStore
from .hot import HotWeights
from .layer import ColdNeurons, _ffn
from .predictor import NeuronPredictor
from .store import ColdSection

HIDDEN = _lib.HIDDEN
REC = fmt.NEURON_RECORD_BYTES


@dataclass
class BatchLayer:
    hot: Optional[HotWeights]
    lut: torch.Tensor                 # (inter,) int32 device: nid -> record slot, -1 hot / absent
    norm_w: torch.Tensor              # (H,) fp16 device
    predictor: Optional[NeuronPredictor]
    section: int                      # section of the file store holding the layer's records


class BatchDecodeStack:
    def __init__(self, layers: list[BatchLayer], store: FileStore, inter: int, eps: float,
                 activation: str = "silu", act_on_both: bool = False, threshold_logit: float = 0.0,
                 device="cuda"):
        self.layers = layers
        self.store = store
        self.inter = inter
        self.eps = float(eps)
        self.activation = activation
        self.act_on_both = act_on_both
        self.thr = float(threshold_logit)
        self.dev = torch.device(device)
        self.n_chunks = (inter + _lib.SEL_CHUNK - 1) // _lib.SEL_CHUNK
        self.cap = max(int(store.n_records[l.section]) for l in layers) if layers else 0
        cap = max(self.cap, 1)
        dev = self.dev
        # selection outputs, per layer parity (a list lives until its FFN)
        self._sel = [dict(slots=torch.empty(self.n_chunks * 256, dtype=torch.int32, device=dev),
                          ids=torch.empty(self.n_chunks * 256, dtype=torch.int32, device=dev),
                          counts=torch.empty(self.n_chunks, dtype=torch.int32, device=dev),
                          dslots=torch.empty(max(inter, 1), dtype=torch.int32, device=dev),
                          dids=torch.empty(max(inter, 1), dtype=torch.int32, device=dev),
                          total=torch.zeros(1, dtype=torch.int32, device=dev))
                     for _ in range(2)]
        self._host_total = [torch.zeros(1, dtype=torch.int32).pin_memory() for _ in range(2)]
        self._host_slots = [torch.empty(max(inter, 1), dtype=torch.int32).pin_memory() for _ in range(2)]
        self._host_ids = [torch.empty(max(inter, 1), dtype=torch.int32).pin_memory() for _ in range(2)]
        self._ring = [torch.empty(cap * REC, dtype=torch.uint8).pin_memory() for _ in range(2)]
        self._stage = [torch.empty((cap, REC), dtype=torch.uint8, device=dev) for _ in range(2)]
        self._arange = torch.arange(cap, dtype=torch.int32, device=dev)
        self._sel_ev = [torch.cuda.Event() for _ in range(2)]
        self._copy_ev = [torch.cuda.Event() for _ in range(2)]
        self._ffn_ev = [torch.cuda.Event() for _ in range(2)]
        self.copy_stream = torch.cuda.Stream(device=dev)
        self._pool = ThreadPoolExecutor(max_workers=1)
        ws = 0
        L = _lib.lib()
        for l in layers:
            if l.predictor is not None:
                ws = max(ws, int(L.oi2_predict_workspace_bytes(ctypes.byref(l.predictor.struct()))))
        self._pws = torch.empty(max(ws, 256), dtype=torch.uint8, device=dev)
        self._nid_cache: dict = {}     # section -> its record nids (this stack's store only)
        self.bytes_read = 0            # record bytes read from the file since construction
        self.trace = None              # set to a list to record (x_in, ids) per layer

    # ── selection (engine.py:274-283) on the device, list back to the host ──
    def _select(self, L: int, x: torch.Tensor, stream):
        lay = self.layers[L]
        S = self._sel[L & 1]
        par = L & 1
        if lay.predictor is None:
            # no predictor: every record of the section, ascending neuron id
            n = int(self.store.n_records[lay.section])
            nids = self._section_nids(lay.section)
            order = np.argsort(nids, kind="stable").astype(np.int32)
            self._host_slots[par][:n] = torch.from_numpy(order)
            self._host_ids[par][:n] = torch.from_numpy(nids[order].astype(np.int32))
            self._host_total[par][0] = n
            with torch.cuda.stream(stream):
                S["total"].fill_(n)
                self._sel_ev[par].record(stream)
            return
        p = lay.predictor.struct()
        Lb = _lib.lib()
        with torch.cuda.stream(stream):
            _lib.check(Lb.oi2_predict_select(
                x.data_ptr(), x.shape[0], lay.norm_w.data_ptr(), ctypes.c_float(self.eps),
                ctypes.byref(p), ctypes.c_float(self.thr), lay.lut.data_ptr(), S["slots"].data_ptr(),
                S["ids"].data_ptr(), S["counts"].data_ptr(), S["dslots"].data_ptr(), S["dids"].data_ptr(),
                S["total"].data_ptr(), self._pws.data_ptr(), self._pws.numel(), stream.cuda_stream or None))
            self._host_total[par].copy_(S["total"], non_blocking=True)
            self._host_slots[par].copy_(S["dslots"], non_blocking=True)
            if self.trace is not None:
                self._host_ids[par].copy_(S["dids"], non_blocking=True)
            self._sel_ev[par].record(stream)

    def _section_nids(self, section: int) -> np.ndarray:
        if section not in self._nid_cache:
            self._nid_cache[section] = self.store.nids(section)
        return self._nid_cache[section]

    def _list(self, L: int):
        """The host copy of layer L's list (waits for its selection)."""
        par = L & 1
        self._sel_ev[par].synchronize()
        n = int(self._host_total[par][0])
        return n, self._host_slots[par][:n].numpy()

    def _read(self, L: int, slots: np.ndarray):
        """Worker thread: layer L's records from the file into pinned buffer
        L & 1, their copy to device buffer L & 1 enqueued on the copy
        stream, then the parity's copy event."""
        n = int(slots.shape[0])
        par = L & 1
        # the pinned buffer was last copied out for layer L - 2
        self._copy_ev[par].synchronize()
        if n:
            self.store.stage(self.layers[L].section, slots, self._ring[par], self._stage[par].view(-1),
                             self.copy_stream)
        self._copy_ev[par].record(self.copy_stream)
        return n

    # ── one step: B tokens through every layer ──
    def decode(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """x (B, H) fp16 on the device; returns the batch after every layer."""
        stream = stream or torch.cuda.current_stream(self.dev)
        n_layers = len(self.layers)
        x = x.to(torch.float16).contiguous()
        self._select(0, x, stream)
        n0, sl0 = self._list(0)
        if self.trace is not None:
            self.trace.clear()
            self.trace.append([x.clone(), self._host_ids[0][:n0].numpy().copy()])
        # the device buffer of a parity was last read by FFN(L - 2): the copy
        # stream waits for it before the worker enqueues the next copies
        self.copy_stream.wait_event(self._ffn_ev[0])
        fut = self._pool.submit(self._read, 0, sl0)
        for L in range(n_layers):
            lay = self.layers[L]
            if L + 1 < n_layers:
                self._select(L + 1, x, stream)
            n = fut.result()
            self.bytes_read += n * REC
            par = L & 1
            cold = None
            if n:
                stream.wait_event(self._copy_ev[par])
                sec = ColdSection(L, np.zeros(0, np.int64), self._stage[par], lay.lut, None, self.inter)
                sec.n_records = n
                cold = ColdNeurons(sec, self._arange, self._sel[par]["total"], 1, max(self.cap, 1),
                                   expected=n)
            with torch.cuda.stream(stream):
                x = _ffn(x, lay.norm_w, self.eps, lay.hot, cold, self.activation, self.act_on_both,
                         add_residual=True)
                self._ffn_ev[par].record(stream)
            if L + 1 < n_layers:
                n1, sl1 = self._list(L + 1)
                if self.trace is not None:
                    self.trace.append([x, self._host_ids[(L + 1) & 1][:n1].numpy().copy()])
                self.copy_stream.wait_event(self._ffn_ev[(L + 1) & 1])
                fut = self._pool.submit(self._read, L + 1, sl1)
        return x

    def close(self):
        self._pool.shutdown(wait=True)
