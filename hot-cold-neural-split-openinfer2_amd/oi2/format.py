"""On-disk cold-record format and the host-side writer.

The byte layout is the split format's contract (splitter.py:23-39, 55-76,
229-256) and is kept identical so that existing ``cold_weights.bin`` /
``cold_index.npy`` files load unchanged:

  section   = 16-byte header ``<HHIq`` (layer u16, expert u16, n_cold u32,
              reserved i64), then n_cold records, then zero padding to a
              4096-byte boundary (splitter.py:230, 250-254)
  record    = ``<H`` neuron id, gate nibbles (H/2 B), up nibbles (H/2 B),
              down nibbles (H/2 B), gate/up/down group scales (32 x fp16 each),
              zero padding to a 64-byte multiple (splitter.py:239-246)
  nibbles   = element 2k in the low nibble, 2k+1 in the high nibble, two's
              complement INT4 (splitter.py:104-106)
  scales    = fp16 absmax/7 per 128-element group (splitter.py:98, 241-243)
  index     = uint64 ``[L, 1, 2]`` of (section byte offset, n_cold)
              (splitter.py:188, 256)

The writer here is vectorised over neurons with numpy instead of the
reference's per-neuron torch loop; the arithmetic (fp32 absmax, fp32 divide,
round-half-even, clamp, fp16 scale storage) is the same and the bytes are
checked against the reference writer's own output.
"""
from __future__ import annotations

import struct

import numpy as np

HIDDEN_DIM = 4096
ALIGN_BYTES = 64
PAGE_ALIGN = 4096
GROUP_SIZE = 128
N_GROUPS = HIDDEN_DIM // GROUP_SIZE              # 32
VEC_BYTES = HIDDEN_DIM // 2                      # 2048
SCALE_BYTES_PER_VEC = N_GROUPS * 2               # 64
SCALE_BYTES_TOTAL = SCALE_BYTES_PER_VEC * 3      # 192
RAW_RECORD = 2 + VEC_BYTES * 3 + SCALE_BYTES_TOTAL   # 6338
NEURON_RECORD_BYTES = ((RAW_RECORD + ALIGN_BYTES - 1) // ALIGN_BYTES) * ALIGN_BYTES  # 6400
SECTION_HEADER_BYTES = 16

# Byte offsets inside one record.
OFF_NID = 0
OFF_GATE = 2
OFF_UP = OFF_GATE + VEC_BYTES                    # 2050
OFF_DOWN = OFF_UP + VEC_BYTES                    # 4098
OFF_SCALES = OFF_DOWN + VEC_BYTES                # 6146
OFF_GATE_SCALES = OFF_SCALES
OFF_UP_SCALES = OFF_SCALES + SCALE_BYTES_PER_VEC     # 6210
OFF_DOWN_SCALES = OFF_SCALES + 2 * SCALE_BYTES_PER_VEC  # 6274

_HEADER = struct.Struct("<HHIq")


def quantize_int4_rows(w: np.ndarray, group_size: int = GROUP_SIZE):
    """Absmax group INT4 quantisation of each row of ``w`` (n, N).

    Row-batched restatement of splitter.py:81-108: scale = max|g| clamped to
    1e-8, divided by 7 in fp32; q = round-half-even(g / scale) clamped to
    [-8, 7]; nibbles packed low-first.  N below the group size is zero padded
    (splitter.py:93-95).  Returns (packed uint8 (n, ceil(N/2)), scales fp32
    (n, n_groups)).
    """
    w = np.asarray(w, dtype=np.float32)
    if w.ndim == 1:
        w = w[None, :]
    n, N = w.shape
    if N % group_size != 0 and N >= group_size:
        raise ValueError(f"tensor length {N} not divisible by group_size {group_size}")
    if N % group_size:
        w = np.concatenate([w, np.zeros((n, group_size - N % group_size), np.float32)], 1)
    g = w.reshape(n, -1, group_size)
    scales = np.maximum(np.abs(g).max(axis=2), np.float32(1e-8)) / np.float32(7.0)
    q = np.clip(np.round(g / scales[:, :, None]), -8, 7).astype(np.int8)
    flat = q.reshape(n, -1)[:, :N]
    if N % 2:
        flat = np.concatenate([flat, np.zeros((n, 1), np.int8)], 1)
    u = flat.view(np.uint8) & np.uint8(0x0F)
    packed = u[:, 0::2] | (u[:, 1::2] << np.uint8(4))
    return packed.astype(np.uint8), scales.astype(np.float32)


def quantize_int4(x, group_size: int = GROUP_SIZE):
    """Single-vector form with the reference signature (splitter.py:81):
    returns (packed bytes, fp32 scales as a numpy array)."""
    packed, scales = quantize_int4_rows(np.asarray(x, np.float32).reshape(1, -1), group_size)
    return packed[0].tobytes(), scales[0]


def build_records(nids, gate, up, down_cols) -> np.ndarray:
    """Encode cold neurons into an (n, 6400) uint8 record array.

    ``gate``/``up`` are (n, H) rows and ``down_cols`` is (n, H): row k is the
    down_proj column of neuron ``nids[k]`` (splitter.py:235-247).
    """
    nids = np.asarray(nids, dtype=np.int64)
    n = nids.shape[0]
    if n and (nids.min() < 0 or nids.max() > 0xFFFF):
        raise ValueError("neuron ids must fit the record's u16 id field")
    rec = np.zeros((n, NEURON_RECORD_BYTES), dtype=np.uint8)
    if n == 0:
        return rec
    rec[:, 0] = (nids & 0xFF).astype(np.uint8)
    rec[:, 1] = ((nids >> 8) & 0xFF).astype(np.uint8)
    for off, soff, w in ((OFF_GATE, OFF_GATE_SCALES, gate), (OFF_UP, OFF_UP_SCALES, up),
                         (OFF_DOWN, OFF_DOWN_SCALES, down_cols)):
        w = np.asarray(w, dtype=np.float32)
        if w.shape != (n, HIDDEN_DIM):
            raise ValueError(f"expected ({n}, {HIDDEN_DIM}) weights, got {w.shape}")
        packed, scales = quantize_int4_rows(w)
        rec[:, off:off + VEC_BYTES] = packed
        rec[:, soff:soff + SCALE_BYTES_PER_VEC] = (
            scales.astype(np.float16).view(np.uint8).reshape(n, SCALE_BYTES_PER_VEC))
    return rec


def section_bytes(layer: int, records: np.ndarray, expert: int = 0) -> bytes:
    """Header + records + page padding for one (layer, expert) section, assuming the
    section starts on a page boundary (splitter.py:229-254)."""
    n = records.shape[0]
    body = _HEADER.pack(layer, expert, n, 0) + records.tobytes()
    pad = (-len(body)) % PAGE_ALIGN
    return body + b"\x00" * pad


class ColdFileWriter:
    """Streams sections into ``cold_weights.bin`` and builds ``cold_index.npy``
    (splitter.py:187-262)."""

    def __init__(self, cold_bin: str, num_layers: int):
        self.path = cold_bin
        self._f = open(cold_bin, "wb")
        self.index = np.zeros((num_layers, 1, 2), dtype=np.uint64)
        self.cursor = 0

    def add_section(self, layer: int, records: np.ndarray):
        data = section_bytes(layer, records)
        self.index[layer, 0] = (self.cursor, records.shape[0])
        self._f.write(data)
        self.cursor += len(data)

    def close(self, cold_index: str):
        self._f.close()
        np.save(cold_index, self.index)
        return self.index
