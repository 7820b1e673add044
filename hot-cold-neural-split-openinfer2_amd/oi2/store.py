"""Cold INT4 neuron store: the split's ``cold_weights.bin`` / ``cold_index.npy``
behind ColdWeightStore's interface (splitter.py:307-407), decoded on the GPU.

The file is memory-mapped as the reference does (splitter.py:322-323).  By
default a layer's section is uploaded to HBM once, on first access, as raw
6400-byte records (the device keeps the INT4 bytes, 16x smaller than the
reference's fp32 tensors); 288 GB of HBM holds a 7B model's ~2.5 GB cold file
many times over.  ``residency="file"`` keeps the reference's model instead:
records are read from the file on every fetch.  ``read_neurons`` keeps the
reference's contract - request order, duplicates kept, absent ids skipped,
None when nothing is found or the section is empty, fp32 (N,H)/(N,H)/(H,N) -
with the dequantisation done by the GPU kernel.  Built with the reference's
three arguments the store returns CPU tensors, as splitter.py:397-403 does;
``device=`` (or ``out_device=``) keeps them on the GPU instead.
"""
from __future__ import annotations

import mmap
import threading

import numpy as np
import torch

from . import _lib
from . import format as fmt


class ColdSection:
    """One (layer, expert) section: records in device or pinned host memory,
    LUT on the device."""

    def __init__(self, layer: int, nids: np.ndarray, records: torch.Tensor, lut: torch.Tensor,
                 lut_host: np.ndarray, inter: int):
        self.layer = layer
        self.nids = nids                  # (n,) int64 on-disk order
        self.records = records            # (n, 6400) uint8, device or pinned host
        self.lut = lut                    # (inter,) int32 device: nid -> slot or -1
        self.lut_host = lut_host
        self.inter = inter
        self.n_records = int(nids.shape[0])
        self._all = None

    def struct(self, gate_bias=None) -> _lib.Cold:
        return _lib.Cold(self.records.data_ptr() if self.n_records else None, self.n_records,
                         _lib.ptr(gate_bias))

    def slots_for(self, neuron_ids) -> np.ndarray:
        """Request-order slots of the ids present in the section."""
        ids = np.asarray(list(neuron_ids) if not isinstance(neuron_ids, np.ndarray) else neuron_ids,
                         dtype=np.int64).reshape(-1)
        ok = (ids >= 0) & (ids < self.inter)
        slots = np.full(ids.shape, -1, dtype=np.int32)
        slots[ok] = self.lut_host[ids[ok]]
        return slots[slots >= 0]

    def all_slots(self) -> torch.Tensor:
        """Every record in ascending neuron-id order (the no-predictor fetch,
        engine.py:282-283)."""
        if self._all is None:
            order = np.argsort(self.nids, kind="stable")
            # a duplicated id resolves to the slot the lut keeps
            keep = self.lut_host[self.nids[order]] == order.astype(np.int32)
            self._all = torch.as_tensor(order[keep].astype(np.int32)).to(self.lut.device)
        return self._all


class ColdWeightStore:
    """splitter.py:307-407.  Where the records live is a choice
    (``residency``):

      * ``"hbm"`` (default): each section's records are copied once out of the
        mapped file into device memory; the FFN kernels gather the active
        ones there (288 GB of HBM holds a 7B model's cold file many times);
      * ``"pinned"`` (or ``pinned=True``): copied once into pinned host memory,
        read by the GPU over PCIe (a decode stack with staging copies the
        active ones into HBM one layer ahead);
      * ``"file"``: the reference's memory model - nothing is copied ahead;
        every fetch reads the requested records from the file (mapped, or
        with ``direct_io=True`` by O_DIRECT page reads) into pinned memory
        and on to the device (liboi2's native file store,
        ``reader_threads`` threads).

    The nid -> slot LUT always lives on the device.

    ``read_neurons`` returns its tensors on ``out_device``: by default the
    CPU when ``device`` is not given (the reference's three-argument form,
    whose tensors are CPU tensors), else ``device``."""

    def __init__(self, cold_bin: str, cold_index: str, config: dict, device=None,
                 pinned: bool = False, residency: str | None = None, direct_io: bool = False,
                 reader_threads: int = 8, out_device=None):
        self.config = config
        self.index = np.load(cold_index)
        self._f = open(cold_bin, "rb")
        size = self._f.seek(0, 2)
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
        self.H = config["hidden_dim"]
        self.I = config.get("intermediate_dim", config.get("expert_inter_dim"))
        if self.H != fmt.HIDDEN_DIM:
            raise ValueError(f"hidden_dim {self.H}: the cold-record layout is sized for "
                             f"{fmt.HIDDEN_DIM}")
        self.device = torch.device(device if device is not None else "cuda")
        self.out_device = torch.device(out_device if out_device is not None
                                       else (device if device is not None else "cpu"))
        self.residency = residency or ("pinned" if pinned else "hbm")
        if self.residency not in ("hbm", "pinned", "file"):
            raise ValueError(f"residency {self.residency!r}: 'hbm', 'pinned' or 'file'")
        self.pinned = self.residency == "pinned"
        self.file = None
        if self.residency == "file":
            from .filestore import FileStore
            self.file = FileStore(cold_bin, cold_index, direct=direct_io, threads=reader_threads)
        self._offset_cache: dict[tuple[int, int], dict[int, int]] = {}
        self._sections: dict[tuple[int, int], ColdSection | None] = {}
        self._lock = threading.Lock()

    # ── reference-compatible pieces ──
    def _section_nids(self, layer_idx: int, expert_idx: int):
        off, n = (int(v) for v in self.index[layer_idx, expert_idx])
        if n == 0:
            return off, None
        base = off + fmt.SECTION_HEADER_BYTES
        raw = np.frombuffer(self._mm, dtype=np.uint8, count=n * fmt.NEURON_RECORD_BYTES,
                            offset=base).reshape(n, fmt.NEURON_RECORD_BYTES)
        nids = raw[:, 0].astype(np.int64) | (raw[:, 1].astype(np.int64) << 8)
        return base, nids

    def _section_offsets(self, layer_idx: int, expert_idx: int):
        """nid -> record byte offset (splitter.py:332-352); None for an empty
        section."""
        key = (layer_idx, expert_idx)
        cached = self._offset_cache.get(key)
        if cached is not None:
            return cached
        base, nids = self._section_nids(layer_idx, expert_idx)
        if nids is None:
            return None
        offs = base + np.arange(nids.shape[0], dtype=np.int64) * fmt.NEURON_RECORD_BYTES
        m = dict(zip(nids.tolist(), offs.tolist()))
        self._offset_cache[key] = m
        return m

    def section(self, layer_idx: int, expert_idx: int = 0) -> ColdSection | None:
        """Copy (once) and return the section's records and device LUT."""
        key = (layer_idx, expert_idx)
        with self._lock:
            if key in self._sections:
                return self._sections[key]
            base, nids = self._section_nids(layer_idx, expert_idx)
            if nids is None:
                self._sections[key] = None
                return None
            self._section_offsets(layer_idx, expert_idx)
            n = nids.shape[0]
            inter = max(int(self.I or 0), int(nids.max()) + 1)
            host = np.frombuffer(self._mm, dtype=np.uint8, count=n * fmt.NEURON_RECORD_BYTES,
                                 offset=base).reshape(n, fmt.NEURON_RECORD_BYTES)
            if self.residency == "file":
                records = None           # read per fetch (fetch_records)
            elif self.pinned:
                records = torch.empty((n, fmt.NEURON_RECORD_BYTES), dtype=torch.uint8,
                                      pin_memory=True)
                records.numpy()[:] = host
            else:
                records = torch.from_numpy(host.copy()).to(self.device)
            lut = np.full(inter, -1, dtype=np.int32)
            # a duplicated id maps to its last record, as the reference's dict does
            uniq, first_rev = np.unique(nids[::-1], return_index=True)
            lut[uniq] = (n - 1 - first_rev).astype(np.int32)
            sec = ColdSection(layer_idx, nids, records, torch.from_numpy(lut).to(self.device),
                              lut, inter)
            sec.file_section = self.file.section_id(layer_idx, expert_idx) if self.file else None
            self._sections[key] = sec
            return sec

    def fetch_records(self, sec: ColdSection, slots, stream) -> "ColdSection":
        """File residency: the records ``slots`` of ``sec`` read from the file
        and copied, in order, into a new device buffer on ``stream``; returns
        a section over them (slot k = the k-th requested record) that carries
        the copy's completion event and keeps its pinned buffer alive until
        the copy has run."""
        s = np.asarray(slots, dtype=np.int32).reshape(-1)
        n = int(s.shape[0])
        host = torch.empty(max(n, 1) * fmt.NEURON_RECORD_BYTES, dtype=torch.uint8, pin_memory=True)
        dst = torch.empty((max(n, 1), fmt.NEURON_RECORD_BYTES), dtype=torch.uint8, device=self.device)
        self.file.stage(sec.file_section, s, host, dst, stream)
        ev = torch.cuda.Event()
        ev.record(stream)
        staged = ColdSection(sec.layer, sec.nids[s] if n else sec.nids[:0], dst, sec.lut, sec.lut_host,
                             sec.inter)
        staged.n_records = n
        staged.event = ev
        staged.host_buffer = host
        return staged

    def read_neurons(self, layer_idx: int, expert_idx: int, neuron_ids):
        """(gate (N,H), up (N,H), down (H,N)) fp32 on ``out_device``, or None
        if the section is empty or no requested id exists
        (splitter.py:354-403)."""
        sec = self.section(layer_idx, expert_idx)
        if sec is None:
            return None
        slots = sec.slots_for(neuron_ids)
        n = int(slots.shape[0])
        if n == 0:
            return None
        dev = self.device
        L = _lib.lib()
        if self.residency == "file":
            stream = torch.cuda.current_stream(dev)
            sec = self.fetch_records(sec, slots, stream)
            slots = np.arange(n, dtype=np.int32)
        gate = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        up = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        down = torch.empty((self.H, n), dtype=torch.float32, device=dev)
        s = torch.as_tensor(slots).to(dev)
        _lib.check(L.oi2_dequant_records(sec.records.data_ptr(), sec.n_records, s.data_ptr(), n,
                                         gate.data_ptr(), up.data_ptr(), down.data_ptr(),
                                         _lib.stream_handle(dev)))
        if self.residency == "file":
            sec.event.synchronize()      # the pinned buffer may be released now
        if self.out_device != dev:
            return gate.to(self.out_device), up.to(self.out_device), down.to(self.out_device)
        return gate, up, down

    def close(self):
        if self.file is not None:
            self.file.close()
        if self._mm is not None:
            self._mm.close()
        self._f.close()
        self._sections.clear()
