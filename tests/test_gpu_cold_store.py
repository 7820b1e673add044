"""The reference's cold-store checks (tests/test_cold_store.py:28-91),
restated and run unchanged in substance against the drop-in
``oi2.ColdWeightStore`` built with the reference's three arguments.

The store decodes on the GPU and, built as the engine builds it
(``ColdWeightStore(cold_bin, cold_index, config)``), returns CPU tensors as
splitter.py:397-403 does, so the reference's exact ``torch.equal``
comparisons against CPU truth apply as written.  The truth vectors are the
INT4 round trip of the fixture's values (tests/common.py:74-81); here they
come from the oracle's dequantisation of the same records, itself pinned
against the SHA-256 of the reference's own truth tensors.
"""
import hashlib
import json
import os
import tempfile

import numpy as np
import pytest
import torch

import oi2
from oracle import oracle as O
from tests.fixtures import synthetic_cold_file

pytestmark = pytest.mark.gpu
H = 4096
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def store_and_truth():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    golden = json.load(open(os.path.join(GOLDEN, "cold_seed0.json")))
    tmp = tempfile.TemporaryDirectory()
    cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp.name, 4, 16, 0)
    raw = open(cold_bin, "rb").read()
    index = np.load(cold_idx)
    truth = {}
    for li in range(4):
        for nid, off in O.section_map(raw, index, li, 0).items():
            _, g, u, d = O.record_vectors(raw, off)
            for name, v in (("gate", g), ("up", u), ("down", d)):
                h = hashlib.sha256(v.astype("<f4").tobytes()).hexdigest()
                assert h == golden["truth_sha256"][f"{li}:{nid}:{name}"], "truth is the reference's"
            truth[(li, nid)] = {"gate": torch.from_numpy(g.astype(np.float32)),
                                "up": torch.from_numpy(u.astype(np.float32)),
                                "down": torch.from_numpy(d.astype(np.float32))}
    store = oi2.ColdWeightStore(cold_bin, cold_idx, config)
    store.paths = (cold_bin, cold_idx)
    yield store, truth
    store.close()
    tmp.cleanup()


def test_readback_values_exact(store_and_truth):
    """tests/test_cold_store.py:28-45: every neuron read alone equals its
    INT4 round trip exactly, with the reference's shapes, on the CPU."""
    store, truth = store_and_truth
    for (li, nid), vecs in truth.items():
        out = store.read_neurons(li, 0, [nid])
        assert out is not None, f"neuron {nid} missing from layer {li}"
        gate, up, down = out
        assert gate.device.type == "cpu" and gate.dtype == torch.float32
        assert gate.shape == (1, H) and up.shape == (1, H) and down.shape == (H, 1)
        assert torch.equal(gate[0], vecs["gate"])
        assert torch.equal(up[0], vecs["up"])
        assert torch.equal(down[:, 0], vecs["down"])


def test_batch_read_shapes_and_order(store_and_truth):
    """tests/test_cold_store.py:48-61."""
    store, truth = store_and_truth
    layer0_ids = sorted(nid for (li, nid) in truth if li == 0)
    gate, up, down = store.read_neurons(0, 0, layer0_ids)
    n = len(layer0_ids)
    assert gate.shape == (n, H) and down.shape == (H, n)
    for row, nid in enumerate(layer0_ids):
        assert torch.equal(gate[row], truth[(0, nid)]["gate"])
        assert torch.equal(down[:, row], truth[(0, nid)]["down"])


def test_missing_ids_skipped_and_all_missing_returns_none(store_and_truth):
    """tests/test_cold_store.py:64-76."""
    store, truth = store_and_truth
    layer0_ids = [nid for (li, nid) in truth if li == 0]
    absent = max(layer0_ids) + 1000
    out = store.read_neurons(0, 0, [layer0_ids[0], absent])
    assert out is not None and out[0].shape[0] == 1
    assert store.read_neurons(0, 0, [absent, absent + 1]) is None


def test_offset_cache_consistency(store_and_truth):
    """tests/test_cold_store.py:79-91."""
    store, truth = store_and_truth
    layer1_ids = [nid for (li, nid) in truth if li == 1][:4]
    first = store.read_neurons(1, 0, layer1_ids)
    assert (1, 0) in store._offset_cache
    second = store.read_neurons(1, 0, layer1_ids)
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_device_output_is_an_opt_in(store_and_truth):
    """out_device keeps the decoded tensors on the GPU (the same bits)."""
    store, truth = store_and_truth
    ids = [nid for (li, nid) in truth if li == 2][:5]
    cpu = store.read_neurons(2, 0, ids)
    gpu_store = oi2.ColdWeightStore(*store.paths, store.config, out_device="cuda:0")
    try:
        dev = gpu_store.read_neurons(2, 0, ids)
        for a, b in zip(cpu, dev):
            assert b.is_cuda and torch.equal(a, b.cpu())
    finally:
        gpu_store.close()
