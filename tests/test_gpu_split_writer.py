"""Device split writer (oi2_quantize_section): the cold half of split_dense
(splitter.py:229-256) with quantize_int4 (splitter.py:81-108).  Bar: the
bytes are identical to the reference writer's -- the golden SHA-256 of the
reference fixture file (tests/common.py:31-104, seed 0), the host writer
over the same inputs at real geometry, and the oracle quantiser on crafted
ties, zero groups, clamp-bound, fp16-subnormal and fp16-overflowing scales."""
import hashlib
import json
import os
import tempfile

import numpy as np
import pytest
import torch

from oi2 import format as fmt
from oi2.split import ColdSectionWriter, quantize_section, quantize_section_rows, section_nbytes
from oracle import oracle as O
from tests.fixtures import synthetic_cold_file

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
H = fmt.HIDDEN_DIM


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a visible GPU"
    return torch.device("cuda:0")


def test_device_writer_reproduces_reference_fixture_file(dev):
    """The seed-0 fixture's 4 layers x 16 unsorted cold neurons written on
    the GPU hash to the reference writer's file."""
    g = json.load(open(os.path.join(GOLDEN, "cold_seed0.json")))
    with tempfile.TemporaryDirectory() as tmp:
        _, _, _, layers = synthetic_cold_file(tmp, 4, 16, 0)
        path = os.path.join(tmp, "gpu_cold.bin")
        w = ColdSectionWriter(path, 4)
        for li in range(4):
            nids, G, U, D = layers[li]
            t = lambda a: torch.as_tensor(a, dtype=torch.float32, device=dev).contiguous()
            sec = quantize_section_rows(li, t(G), t(U), t(D), nids)
            w.add_section_bytes(li, len(nids), sec)
        index = w.close(os.path.join(tmp, "gpu_index.npy"))
        raw = open(path, "rb").read()
    assert len(raw) == g["file_bytes"]
    assert index.reshape(-1).tolist() == g["cold_index"]
    assert hashlib.sha256(raw).hexdigest() == g["file_sha256"]


def test_device_writer_full_matrices_match_host_writer(dev):
    """gate/up (I, H) rows and strided down (H, I) columns of a layer, the
    cold ids ascending as split_dense writes them, against the host writer."""
    gen = torch.Generator(device=dev).manual_seed(3)
    inter = 2048
    gate = torch.randn((inter, H), generator=gen, device=dev) * 0.02
    up = torch.randn((inter, H), generator=gen, device=dev) * 0.02
    down = torch.randn((H, inter), generator=gen, device=dev) * 0.02
    cold = np.sort(torch.randperm(inter, generator=gen, device=dev)[:1500].cpu().numpy())
    sec = quantize_section(5, gate, up, down, cold).cpu().numpy()
    g, u, d = gate.cpu().numpy(), up.cpu().numpy(), down.cpu().numpy()
    ref = fmt.section_bytes(5, fmt.build_records(cold, g[cold], u[cold], d[:, cold].T))
    assert sec.nbytes == len(ref) == section_nbytes(len(cold))
    assert sec.tobytes() == ref


def _crafted_vectors():
    rng = np.random.default_rng(11)
    vs = []
    v = np.zeros(H, np.float32)            # every group all zero: scale 1e-8 / 7, q = 0
    vs.append(v)
    v = rng.standard_normal(H).astype(np.float32)
    g = v.reshape(-1, 128)
    g[:, 0] = 7.0                          # scale exactly 1: x.5 values are ties
    g[:, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 6.5, -6.5]
    vs.append(v)
    vs.append((rng.standard_normal(H) * 1e-9).astype(np.float32))   # max below the 1e-8 clamp
    vs.append((rng.standard_normal(H) * 1e-5).astype(np.float32))   # fp16-subnormal scales
    vs.append((rng.standard_normal(H) * 1e6).astype(np.float32))    # scale overflows fp16 (inf)
    v = rng.standard_normal(H).astype(np.float32)
    v.reshape(-1, 128)[:, 5] = -np.abs(v.reshape(-1, 128)).max(1) * 1.0   # negative absmax
    vs.append(v)
    return np.stack(vs)


def test_device_quantiser_matches_oracle_on_edge_values(dev):
    vecs = _crafted_vectors()
    n = vecs.shape[0]
    t = torch.as_tensor(vecs, device=dev)
    nids = np.arange(100, 100 + n)
    sec = quantize_section_rows(0, t, t.flip(0).contiguous(), t.roll(1, 0).contiguous(), nids)
    rec = sec.cpu().numpy()[16:16 + n * fmt.NEURON_RECORD_BYTES].reshape(n, -1)
    for k in range(n):
        for m, src in enumerate((vecs[k], vecs[n - 1 - k], vecs[(k - 1) % n])):
            packed, scales = O.quantize_int4_ref(src)
            off = fmt.OFF_GATE + m * fmt.VEC_BYTES
            soff = fmt.OFF_SCALES + m * fmt.SCALE_BYTES_PER_VEC
            assert rec[k, off:off + fmt.VEC_BYTES].tobytes() == bytes(packed), (k, m)
            assert (rec[k, soff:soff + fmt.SCALE_BYTES_PER_VEC].tobytes()
                    == np.asarray(scales, np.float32).astype(np.float16).tobytes()), (k, m)
        assert int(rec[k, 0]) | (int(rec[k, 1]) << 8) == nids[k]
        assert not rec[k, fmt.RAW_RECORD:].any()


def test_device_writer_empty_section(dev):
    z = torch.zeros((0, H), dtype=torch.float32, device=dev)
    sec = quantize_section_rows(7, z, z, z, [])
    assert sec.cpu().numpy().tobytes() == fmt.section_bytes(7, np.zeros((0, fmt.NEURON_RECORD_BYTES), np.uint8))
