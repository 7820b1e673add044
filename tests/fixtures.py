"""Seeded input builders shared by the tests.

``synthetic_cold_file`` restates the reference fixture
tests/common.py:31-104 (same torch RNG consumption order: per layer one
randperm for the ids, per neuron three randn(4096)), writing through the
library's own record writer; its byte image is compared against the golden
hash recorded from the reference.
"""
import os

import numpy as np
import torch

from oi2 import format as fmt


def synthetic_cold_file(out_dir, num_layers=4, n_cold=16, seed=0):
    torch.manual_seed(seed)
    os.makedirs(out_dir, exist_ok=True)
    cold_bin = os.path.join(out_dir, "cold_weights.bin")
    cold_idx = os.path.join(out_dir, "cold_index.npy")
    w = fmt.ColdFileWriter(cold_bin, num_layers)
    layers = {}
    for li in range(num_layers):
        nids = torch.randperm(n_cold * 3)[:n_cold].tolist()
        vecs = []
        for _ in nids:
            g = torch.randn(fmt.HIDDEN_DIM)
            u = torch.randn(fmt.HIDDEN_DIM)
            d = torch.randn(fmt.HIDDEN_DIM)
            vecs.append((g.numpy(), u.numpy(), d.numpy()))
        G = np.stack([v[0] for v in vecs]) if vecs else np.zeros((0, fmt.HIDDEN_DIM), np.float32)
        U = np.stack([v[1] for v in vecs]) if vecs else np.zeros((0, fmt.HIDDEN_DIM), np.float32)
        D = np.stack([v[2] for v in vecs]) if vecs else np.zeros((0, fmt.HIDDEN_DIM), np.float32)
        w.add_section(li, fmt.build_records(nids, G, U, D))
        layers[li] = (nids, G, U, D)
    w.close(cold_idx)
    config = {"hidden_dim": fmt.HIDDEN_DIM, "intermediate_dim": n_cold * 3}
    return cold_bin, cold_idx, config, layers
