"""Cold INT4 neuron store: the split's ``cold_weights.bin`` / ``cold_index.npy``
behind ColdWeightStore's interface (splitter.py:307-407), decoded on the GPU.

The file is memory-mapped as the reference does (splitter.py:322-323).  A
layer's section is uploaded to HBM once, on first access, as raw 6400-byte
records (the device keeps the INT4 bytes, 16x smaller than the reference's
fp32 tensors); 288 GB of HBM holds a 7B model's ~2.5 GB cold file many times
over.  ``read_neurons`` keeps the reference's contract - request order,
duplicates kept, absent ids skipped, None when nothing is found or the section
is empty, fp32 (N,H)/(N,H)/(H,N) - but returns device tensors produced by the
dequant kernel.
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
    """splitter.py:307-407 with a section cache: each section's records are
    copied once out of the mapped file, into device memory, or with
    ``pinned=True`` into pinned host memory (read by the GPU over PCIe; a
    decode stack with staging copies the active ones into HBM one layer
    ahead).  The nid -> slot LUT always lives on the device."""

    def __init__(self, cold_bin: str, cold_index: str, config: dict, device="cuda",
                 pinned: bool = False):
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
        self.device = torch.device(device)
        self.pinned = bool(pinned)
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
            if self.pinned:
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
            self._sections[key] = sec
            return sec

    def read_neurons(self, layer_idx: int, expert_idx: int, neuron_ids):
        """(gate (N,H), up (N,H), down (H,N)) fp32 on the store's device, or
        None if the section is empty or no requested id exists."""
        sec = self.section(layer_idx, expert_idx)
        if sec is None:
            return None
        slots = sec.slots_for(neuron_ids)
        n = int(slots.shape[0])
        if n == 0:
            return None
        dev = self.device
        L = _lib.lib()
        gate = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        up = torch.empty((n, self.H), dtype=torch.float32, device=dev)
        down = torch.empty((self.H, n), dtype=torch.float32, device=dev)
        s = torch.as_tensor(slots).to(dev)
        _lib.check(L.oi2_dequant_records(sec.records.data_ptr(), sec.n_records, s.data_ptr(), n,
                                         gate.data_ptr(), up.data_ptr(), down.data_ptr(),
                                         _lib.stream_handle(dev)))
        return gate, up, down

    def close(self):
        if self._mm is not None:
            self._mm.close()
        self._f.close()
        self._sections.clear()
