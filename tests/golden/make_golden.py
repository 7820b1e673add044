"""Write the golden vectors for the cold-record writer from the reference itself.

Run once, in the build container where the reference checkout exists:

    python tests/golden/make_golden.py /root/reference

Only the writer side is imported (``splitter.quantize_int4`` and the test
fixture ``tests/common.py:build_synthetic_cold_file``), because the byte image
those produce is the one thing on the path that closed forms and invariants do
not fix: RNG consumption order, fp32 scale rounding, fp16 scale storage and the
exact packing.  Everything else on the path (dequant, FFN, predictor) is pinned
without running the reference.

Outputs (all small):
  cold_seed0.json        sha256 of cold_weights.bin and of every truth vector of
                         build_synthetic_cold_file(num_layers=4, n_cold=16, seed=0),
                         the cold_index table and the on-disk nid order
  cold_seed0_records.npy the first two raw 6400-byte records of every section
  quant_edge.json        quantize_int4 packed bytes and fp32 scales for crafted
                         inputs (ties, zeros, short vectors, large values)
"""
import hashlib
import importlib.util
import json
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _load(ref_root, name, rel):
    spec = importlib.util.spec_from_file_location(name, os.path.join(ref_root, rel))
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


def main(ref_root):
    sys.path.insert(0, ref_root)
    splitter = _load(ref_root, "splitter", "splitter.py")
    common = _load(ref_root, "ref_tests_common", "tests/common.py")

    # 1. synthetic cold file, seed 0, the reference fixture's default geometry
    with tempfile.TemporaryDirectory() as tmp:
        cold_bin, cold_idx, config, truth = common.build_synthetic_cold_file(
            tmp, num_layers=4, n_cold=16, seed=0)
        raw = open(cold_bin, "rb").read()
        index = np.load(cold_idx)
    rec = splitter.NEURON_RECORD_BYTES
    order = {}
    samples = []
    for li in range(index.shape[0]):
        off, n = int(index[li, 0, 0]), int(index[li, 0, 1])
        nids = [int.from_bytes(raw[off + 16 + k * rec: off + 18 + k * rec], "little")
                for k in range(n)]
        order[str(li)] = nids
        for k in range(2):
            s = off + 16 + k * rec
            samples.append(np.frombuffer(raw[s:s + rec], dtype=np.uint8))
    truth_sha = {}
    for (li, nid), vecs in sorted(truth.items()):
        for name in ("gate", "up", "down"):
            arr = vecs[name].numpy().astype("<f4")
            truth_sha[f"{li}:{nid}:{name}"] = hashlib.sha256(arr.tobytes()).hexdigest()
    out = {
        "num_layers": 4, "n_cold": 16, "seed": 0,
        "file_bytes": len(raw),
        "file_sha256": hashlib.sha256(raw).hexdigest(),
        "cold_index": index.reshape(-1).tolist(),
        "nid_order": order,
        "config": config,
        "truth_sha256": truth_sha,
        "torch_version": torch.__version__,
    }
    with open(os.path.join(HERE, "cold_seed0.json"), "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    np.save(os.path.join(HERE, "cold_seed0_records.npy"), np.stack(samples))

    # 2. quantize_int4 on crafted inputs
    cases = {
        "ties_one_group": torch.tensor([7.0, 3.5, -3.5, 2.5, -2.5, 0.5, -0.5, 1.5] * 16),
        "zeros": torch.zeros(256),
        "short_100": torch.linspace(-3.0, 2.0, 100),
        "extreme": torch.tensor([100.0, -100.0, 50.0, -50.0] * 32),
        "tiny": torch.full((128,), 1e-9),
        "mixed_groups": torch.cat([torch.arange(128, dtype=torch.float32) - 64.0,
                                   torch.ones(128) * -0.25]),
    }
    g = torch.Generator().manual_seed(7)
    cases["randn_4096"] = torch.randn(4096, generator=g) * 3.0
    qout = {}
    for name, x in cases.items():
        packed, scales = splitter.quantize_int4(x.clone())
        qout[name] = {
            "x_f32_hex": x.numpy().astype("<f4").tobytes().hex(),
            "packed_hex": packed.hex(),
            "scales_f32_hex": scales.numpy().astype("<f4").tobytes().hex(),
            "scales_f16_hex": scales.to(torch.float16).numpy().tobytes().hex(),
        }
    with open(os.path.join(HERE, "quant_edge.json"), "w") as f:
        json.dump(qout, f, indent=1, sort_keys=True)
    print("wrote golden vectors to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
