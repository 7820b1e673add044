"""Cold records read from the split file on every request (liboi2's native
file store): ColdWeightStore's mmap and per-record slicing
(splitter.py:317-403) without its per-neuron Python loop or dequantisation.

``FileStore.read`` copies the requested records of one section, whole and in
request order, into a host buffer - normally pinned, so that one
``hipMemcpyAsync`` moves the batch to the device, where the FFN kernels decode
the INT4 themselves.  Reads go either through a mapping of the file (the page
cache) or, with ``direct=True``, through O_DIRECT page reads that bypass it.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from . import format as fmt


class FileStore:
    def __init__(self, cold_bin: str, cold_index: str, direct: bool = False, threads: int = 8,
                 read_gap: int | None = None):
        index = np.load(cold_index)
        self.n_experts = int(index.shape[1]) if index.ndim == 3 else 1
        flat = np.ascontiguousarray(index.reshape(-1, 2).astype(np.uint64))
        self.sections = int(flat.shape[0])
        self.n_records = flat[:, 1].astype(np.int64)
        self.offsets = flat[:, 0].astype(np.int64)
        self.direct = bool(direct)
        self._index = flat
        h = ctypes.c_void_p()
        L = _lib.load_library()
        rc = L.oi2_file_store_open(cold_bin.encode(), flat.ctypes.data, self.sections,
                                   int(self.direct), int(threads), ctypes.byref(h))
        _lib.check(rc)
        self._h = h
        if read_gap is not None:
            _lib.check(L.oi2_file_store_set_read_gap(h, int(read_gap)))

    def section_id(self, layer: int, expert: int = 0) -> int:
        return layer * self.n_experts + expert

    def nids(self, section: int) -> np.ndarray:
        """The section's neuron ids in file order (each record's leading u16)."""
        n = int(self.n_records[section])
        if n == 0:
            return np.zeros(0, np.int64)
        rec = np.empty((n, fmt.NEURON_RECORD_BYTES), np.uint8)
        self.read(section, np.arange(n, dtype=np.int32), rec)
        return rec[:, 0].astype(np.int64) | (rec[:, 1].astype(np.int64) << 8)

    def read(self, section: int, slots, out):
        """Records ``slots`` of ``section`` into ``out`` (a host numpy array or
        CPU tensor of at least len(slots) x 6400 bytes, contiguous), request
        order; returns the number of records written."""
        s = np.ascontiguousarray(np.asarray(slots, dtype=np.int32).reshape(-1))
        n = int(s.shape[0])
        if torch.is_tensor(out):
            if out.is_cuda or not out.is_contiguous() or out.dtype != torch.uint8:
                raise ValueError("out must be a contiguous uint8 host tensor")
            ptr, nbytes = out.data_ptr(), out.numel()
        else:
            if not out.flags["C_CONTIGUOUS"] or out.dtype != np.uint8:
                raise ValueError("out must be a C-contiguous uint8 array")
            ptr, nbytes = out.ctypes.data, out.nbytes
        if nbytes < n * fmt.NEURON_RECORD_BYTES:
            raise ValueError(f"out holds {nbytes} bytes; {n} records need {n * fmt.NEURON_RECORD_BYTES}")
        _lib.check(_lib.load_library().oi2_file_store_read(self._h, int(section), s.ctypes.data, n, ptr))
        return n

    def stage(self, section: int, slots, host_buf: torch.Tensor, dst: torch.Tensor, stream) -> int:
        """Read the records into ``host_buf`` (pinned) and enqueue their copy
        to ``dst`` (device, contiguous) on ``stream``; returns the count.
        ``host_buf`` must stay untouched until the copy has run."""
        s = np.ascontiguousarray(np.asarray(slots, dtype=np.int32).reshape(-1))
        n = int(s.shape[0])
        need = n * fmt.NEURON_RECORD_BYTES
        if host_buf.numel() < need or dst.numel() < need or not dst.is_cuda or host_buf.is_cuda:
            raise ValueError(f"{n} records need {need} bytes of pinned host and device buffer")
        _lib.check(_lib.load_library().oi2_file_store_stage(
            self._h, int(section), s.ctypes.data, n, host_buf.data_ptr(), dst.data_ptr(),
            stream.cuda_stream or None))
        return n

    def close(self):
        if self._h:
            _lib.load_library().oi2_file_store_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
