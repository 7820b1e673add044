"""The allocation-free decode FFN entry point (oi2_ffn_forward_noalloc)
against oi2_ffn_forward, through the C ABI: two calls in a row on the same
GPU (so the second finds the first's contents in the shared static scratch),
the second on a smaller input; both equal to the workspace entry point bit
for bit (the same kernels and launch shapes) and within the FFN bar of the
float64 oracle.  Requests past the scratch's limits are refused before any
launch."""
import ctypes

import numpy as np
import pytest
import torch

import oi2
from oi2 import _lib
from oi2.layer import ColdNeurons, _ffn
from oi2.store import ColdSection
from oi2.synth import SyntheticLayer
from oracle import oracle as O
from tests.gpu_helpers import EPS, assert_ffn_close, cold_dense, hot_dense, normed_f16

pytestmark = pytest.mark.gpu
H = 4096


def _section(lay):
    return ColdSection(0, lay.cold_ids.cpu().numpy(), lay.records, lay.lut, lay.lut.cpu().numpy(),
                       lay.inter)


def _noalloc(x, lay, cold, activation="silu", both=False, add_residual=True):
    L = _lib.lib()
    dev = x.device
    B = x.shape[0]
    hot_s = lay.hot.struct()
    cold_s, act_s = cold.structs()
    out = torch.empty_like(x)
    y32 = torch.empty((B, H), dtype=torch.float32, device=dev)
    rc = L.oi2_ffn_forward_noalloc(x.data_ptr(), B, lay.norm_w.data_ptr(), ctypes.c_float(EPS),
                                   ctypes.byref(hot_s), ctypes.byref(cold_s), ctypes.byref(act_s),
                                   _lib.ACT_RELU if activation == "relu" else _lib.ACT_SILU,
                                   int(both), int(add_residual), out.data_ptr(), y32.data_ptr(),
                                   _lib.stream_handle(dev))
    _lib.check(rc)
    return out, y32


def test_noalloc_matches_workspace_entry_point_twice():
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(71)
    L = _lib.lib()
    assert L.oi2_ffn_noalloc_max_expected() == 1024
    assert L.oi2_ffn_noalloc_scratch_bytes() >= (4096 + 256 * 4096) * 4
    big = SyntheticLayer(g, 14336, 3584, device=dev)
    small = SyntheticLayer(g, 2048, 500, device=dev)
    cases = [(big, 900, 2, "silu", False), (small, 100, 1, "relu", True)]   # second call smaller
    results = []
    for lay, n_act, B, activation, both in cases:
        n_cold = lay.records.shape[0]
        slots = torch.randperm(n_cold, generator=g, device=dev)[:n_act].int()
        cold = ColdNeurons.from_slots(_section(lay), slots)
        x = torch.randn((B, H), generator=g, device=dev).half()
        out, y32 = _noalloc(x, lay, cold, activation, both)
        torch.cuda.synchronize()
        results.append((lay, slots, cold, x, out.clone(), y32.clone(), activation, both))
    for lay, slots, cold, x, out, y32, activation, both in results:
        B = x.shape[0]
        # the workspace entry point on each token alone runs the same kernels
        for b in range(B):
            o_ref, y_ref = _ffn(x[b:b + 1], lay.norm_w, EPS, lay.hot, cold, activation, both,
                                add_residual=True, want_y32=True)
            torch.cuda.synchronize()
            assert torch.equal(y32[b], y_ref[0]) and torch.equal(out[b], o_ref[0])
        if B > 1:   # and its batch path (matrix cores) agrees to rounding
            _, y_b = _ffn(x, lay.norm_w, EPS, lay.hot, cold, activation, both, add_residual=True,
                          want_y32=True)
            assert_ffn_close(y32.cpu().numpy().ravel(), y_b.cpu().numpy().ravel(), tol=2e-3,
                             cos_min=0.99999, what="noalloc vs batch path")
        xn = normed_f16(x, lay.norm_w)
        ref = O.sparse_ffn(xn, activation, both, *hot_dense(lay.hot), *cold_dense(lay.records, slots))
        for b in range(B):
            assert_ffn_close(y32[b].cpu().numpy(), ref[b], what=f"noalloc row {b}")


def test_noalloc_refuses_past_its_limits():
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(72)
    lay = SyntheticLayer(g, 14336, 3584, device=dev)
    slots = torch.arange(5000, dtype=torch.int32, device=dev)
    cold = ColdNeurons.from_slots(_section(lay), slots)        # expected = capacity = 5000
    x = torch.randn((1, H), generator=g, device=dev).half()
    with pytest.raises(oi2.OI2Error, match="static scratch"):
        _noalloc(x, lay, cold)
    cold.expected = 1000                                       # within the limit: runs
    out, y32 = _noalloc(x, lay, cold)
    _, y_ref = _ffn(x, lay.norm_w, EPS, lay.hot, cold, "silu", False, add_residual=True,
                    want_y32=True)
    torch.cuda.synchronize()
    assert torch.equal(y32, y_ref)
