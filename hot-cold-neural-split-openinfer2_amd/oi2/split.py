"""Device-side writer for the cold half of the split format.

split_dense (splitter.py:187-262) walks each layer's cold neurons in a
Python loop, quantising three vectors per neuron with quantize_int4
(splitter.py:81-108) and writing the record bytes one by one.  Here a layer's
whole section (header, records, page padding) is produced by one call of
``oi2_quantize_section`` on the GPU from the layer's fp32 weights, and the
byte image is identical to the reference writer's.

``ColdSectionWriter`` streams such sections into ``cold_weights.bin`` and
builds ``cold_index.npy`` the way split_dense does (splitter.py:187-188,
229-256).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .format import HIDDEN_DIM


def section_nbytes(n_cold: int) -> int:
    """Bytes of a section holding n_cold records (header + records + padding)."""
    return int(_lib.load_library().oi2_section_bytes(int(n_cold)))


def quantize_section(layer: int, gate: torch.Tensor, up: torch.Tensor, down: torch.Tensor,
                     cold_ids, expert: int = 0, nids=None) -> torch.Tensor:
    """One layer's section of cold_weights.bin as a uint8 device tensor.

    ``gate``/``up`` are the model's (I, H) projections and ``down`` its
    (H, I) projection, fp32 on the GPU; ``cold_ids`` are the cold neurons in
    the order their records are written (split_dense writes ascending ids,
    splitter.py:215, 234).  Record k quantises gate[id], up[id] and
    down[:, id] (splitter.py:235-237).  ``nids``, when given, replaces the
    ids stored in the records (the default is cold_ids itself).  For vectors
    that are already gathered per neuron see :func:`quantize_section_rows`.
    """
    dev = gate.device
    for name, t in (("gate", gate), ("up", up), ("down", down)):
        if t.dtype != torch.float32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 tensor on {dev}")
    inter, hidden = gate.shape
    if hidden != HIDDEN_DIM or up.shape != gate.shape or down.shape != (hidden, inter):
        raise ValueError(f"expected gate/up ({inter}, {HIDDEN_DIM}) and down ({HIDDEN_DIM}, {inter})")
    rows = torch.as_tensor(np.asarray(list(cold_ids), np.int64), device=dev)
    if rows.numel() and (int(rows.min()) < 0 or int(rows.max()) >= inter):
        raise ValueError("cold ids out of range")
    return _run(layer, expert, gate, up, down, rows, nids if nids is not None else rows,
                (hidden, hidden, 1), (1, 1, inter))


def quantize_section_rows(layer: int, gate: torch.Tensor, up: torch.Tensor, down_cols: torch.Tensor,
                          nids, expert: int = 0) -> torch.Tensor:
    """The same section from pre-gathered vectors: row k of gate, up and
    down_cols (each (n, H) fp32) are neuron nids[k]'s gate row, up row and
    down column."""
    dev = gate.device
    for name, t in (("gate", gate), ("up", up), ("down_cols", down_cols)):
        if t.dtype != torch.float32 or t.device != dev or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous fp32 tensor on {dev}")
        if t.dim() != 2 or t.shape[1] != HIDDEN_DIM or t.shape[0] != gate.shape[0]:
            raise ValueError(f"{name} must be (n, {HIDDEN_DIM})")
    n = gate.shape[0]
    rows = torch.arange(n, device=dev, dtype=torch.int64)
    return _run(layer, expert, gate, up, down_cols, rows, nids,
                (HIDDEN_DIM, HIDDEN_DIM, HIDDEN_DIM), (1, 1, 1))


def _run(layer, expert, gate, up, down, rows, nids, row_stride, elem_stride):
    L = _lib.lib()
    dev = gate.device
    n = int(rows.numel())
    ids = np.asarray(torch.as_tensor(nids).cpu().numpy() if torch.is_tensor(nids) else list(nids),
                     np.int64).reshape(-1)
    if ids.size != n:
        raise ValueError("one id per record is required")
    if n and (ids.min() < 0 or ids.max() > 0xFFFF):
        raise ValueError("neuron ids must fit the record's u16 id field")
    nid16 = torch.as_tensor(ids.astype(np.uint16).view(np.int16), device=dev)
    rows32 = rows.to(torch.int32)
    size = int(L.oi2_section_bytes(n))
    out = torch.empty(size, dtype=torch.uint8, device=dev)
    rs = (ctypes.c_int64 * 3)(*row_stride)
    es = (ctypes.c_int64 * 3)(*elem_stride)
    _lib.check(L.oi2_quantize_section(int(layer), int(expert), n, _lib.ptr(nid16), _lib.ptr(rows32),
                                      _lib.ptr(gate), _lib.ptr(up), _lib.ptr(down),
                                      ctypes.cast(rs, ctypes.c_void_p), ctypes.cast(es, ctypes.c_void_p),
                                      _lib.ptr(out), size, _lib.stream_handle(dev)))
    return out


class ColdSectionWriter:
    """cold_weights.bin + cold_index.npy from device-built sections
    (splitter.py:187-188, 229-256)."""

    def __init__(self, cold_bin: str, num_layers: int):
        self.path = cold_bin
        self._f = open(cold_bin, "wb")
        self.index = np.zeros((num_layers, 1, 2), dtype=np.uint64)
        self.cursor = 0

    def add_layer(self, layer: int, gate, up, down, cold_ids):
        sec = quantize_section(layer, gate, up, down, cold_ids)
        return self.add_section_bytes(layer, len(list(cold_ids)), sec)

    def add_section_bytes(self, layer: int, n_cold: int, section: torch.Tensor):
        data = section.cpu().numpy().tobytes()
        self.index[layer, 0] = (self.cursor, n_cold)
        self._f.write(data)
        self.cursor += len(data)
        return len(data)

    def close(self, cold_index: str):
        self._f.close()
        np.save(cold_index, self.index)
        return self.index
