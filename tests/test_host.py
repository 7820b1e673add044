"""Host-side logic and the C ABI's exported surface.  CPU only: nothing here
launches a kernel."""
import os
import re
import tempfile

import numpy as np
import pytest
import torch

import oi2
from oi2 import _lib
from oi2 import format as fmt
from oi2.synth import quantize_int4_rows_torch, records_from_rows
from oracle import oracle as O
from tests.fixtures import synthetic_cold_file

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "oi2.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(oi2_[a-z_0-9]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    lib = oi2.load_library()
    names = _header_functions()
    assert len(names) >= 14
    for n in names:
        assert hasattr(lib, n), f"liboi2.so does not export {n}"
    assert set(names) <= set(_lib._SIGS), "ctypes signatures missing for some entry points"
    assert lib.oi2_abi_version() == _lib.ABI_VERSION == 2
    assert lib.oi2_record_bytes() == fmt.NEURON_RECORD_BYTES == 6400


def test_argument_validation_without_gpu():
    """Bad arguments are rejected on the host with a message, before any
    device work."""
    lib = oi2.load_library()
    rc = lib.oi2_dequant_records(None, 0, None, 5, None, None, None, None)
    assert rc == 1
    assert b"null" in lib.oi2_last_error()
    p = _lib.Predictor(100, 12, 0, 1, 1, 1)       # rank not a multiple of 8
    import ctypes
    rc = lib.oi2_predict(1, _lib.DTYPE_F16, 1, ctypes.byref(p), 0.0, None, None, None, None, 0, None)
    assert rc == 1 and b"rank" in lib.oi2_last_error()
    rc = lib.oi2_predict(1, 7, 1, ctypes.byref(p), 0.0, None, None, None, None, 0, None)
    assert rc == 1 and b"h_dtype" in lib.oi2_last_error()
    assert lib.oi2_ffn_workspace_bytes(1, 3584, 14336) >= (3584 + 2 * 14336 + 2048) * 4


def test_split_writer_host_side():
    """Section size is the reference writer's framing (16-byte header, 6400
    per record, padding to 4096; splitter.py:229-254), and bad arguments are
    rejected before any device work."""
    lib = oi2.load_library()
    for n in (0, 1, 16, 639, 640, 10752):
        body = 16 + 6400 * n
        assert lib.oi2_section_bytes(n) == (body + 4095) // 4096 * 4096
        assert lib.oi2_section_bytes(n) == len(fmt.section_bytes(0, np.zeros((n, 6400), np.uint8)))
    assert lib.oi2_section_bytes(-1) == 0
    assert lib.oi2_quantize_section(0, 0, -1, None, None, None, None, None, None, None, None, 0,
                                    None) == 1
    assert b"non-negative" in lib.oi2_last_error()
    assert lib.oi2_quantize_section(70000, 0, 0, None, None, None, None, None, None, None, None, 0,
                                    None) == 1
    assert lib.oi2_quantize_section(0, 0, 1, None, None, None, None, None, None, None, 64, 4096,
                                    None) == 1   # section smaller than one record needs
    assert b"smaller" in lib.oi2_last_error()


def test_compute_entry_points_fail_loudly_without_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(oi2.OI2Error):
        _lib.lib()


def test_format_constants_match_reference_layout():
    assert fmt.RAW_RECORD == 6338
    assert (fmt.OFF_GATE, fmt.OFF_UP, fmt.OFF_DOWN, fmt.OFF_SCALES) == (2, 2050, 4098, 6146)
    assert fmt.OFF_DOWN_SCALES + fmt.SCALE_BYTES_PER_VEC == fmt.RAW_RECORD


def test_torch_record_writer_matches_numpy_writer():
    g = torch.Generator().manual_seed(5)
    n = 9
    G, U, D = (torch.randn((n, 4096), generator=g) * s for s in (0.02, 1.0, 3.0))
    G[3] = 0.0                                   # all-zero row: scale clamps to 1e-8/7
    U[4, :128] = torch.tensor([7.0, 3.5, -3.5, 0.5] * 32)   # exact .5 ties
    nids = torch.tensor([5, 300, 65535, 0, 17, 2, 9, 11, 40000])
    a = records_from_rows(nids, G, U, D).numpy()
    b = fmt.build_records(nids.numpy(), G.numpy(), U.numpy(), D.numpy())
    assert np.array_equal(a, b)
    p, s = quantize_int4_rows_torch(U)
    for r in range(n):
        pr, sr = O.quantize_int4_ref(U[r].numpy())
        assert p[r].numpy().tobytes() == pr and np.array_equal(s[r].numpy(), sr)


def test_store_host_logic_on_golden_file():
    """ColdWeightStore's section map, LUT and request-order slot lookup
    (splitter.py:332-372) on the reference fixture's byte image."""
    with tempfile.TemporaryDirectory() as tmp:
        cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp, 4, 16, 0)
        store = oi2.ColdWeightStore(cold_bin, cold_idx, config, device="cpu")
        raw = open(cold_bin, "rb").read()
        index = np.load(cold_idx)
        try:
            for li in range(4):
                assert store._section_offsets(li, 0) == O.section_map(raw, index, li, 0)
                sec = store.section(li)
                nids = layers[li][0]
                assert sec.nids.tolist() == nids
                assert sec.n_records == 16
                req = [nids[7], 10_000, nids[2], nids[7], -3, nids[15]]
                assert sec.slots_for(req).tolist() == [7, 2, 7, 15]
                assert sec.slots_for([10_000]).size == 0
                order = sec.all_slots().tolist()
                assert [nids[s] for s in order] == sorted(nids)
                assert np.array_equal(sec.records.numpy()[3],
                                      np.frombuffer(raw, np.uint8,
                                                    count=6400, offset=int(index[li, 0, 0]) + 16 + 3 * 6400))
            assert (1, 0) in store._offset_cache
        finally:
            store.close()


def test_store_duplicate_ids_resolve_to_last_record():
    with tempfile.TemporaryDirectory() as tmp:
        w = fmt.ColdFileWriter(os.path.join(tmp, "c.bin"), 2)
        rng = np.random.default_rng(0)
        rows = rng.standard_normal((4, 4096)).astype(np.float32)
        w.add_section(0, fmt.build_records([3, 8, 3, 5], rows, rows, rows))
        w.add_section(1, fmt.build_records([], np.zeros((0, 4096)), np.zeros((0, 4096)),
                                           np.zeros((0, 4096))))
        w.close(os.path.join(tmp, "i.npy"))
        store = oi2.ColdWeightStore(os.path.join(tmp, "c.bin"), os.path.join(tmp, "i.npy"),
                                    {"hidden_dim": 4096, "intermediate_dim": 16}, device="cpu")
        try:
            sec = store.section(0)
            assert sec.slots_for([3, 5, 8]).tolist() == [2, 3, 1]
            assert store._section_offsets(0, 0)[3] == 16 + 2 * 6400
            assert store.section(1) is None
            assert store._section_offsets(1, 0) is None
            assert store.read_neurons(1, 0, [1, 2]) is None
        finally:
            store.close()


def test_logit_threshold_equivalence():
    for p in (0.5, 0.05, 0.95, 0.3):
        t = _lib.logit_threshold(p)
        assert abs(1 / (1 + np.exp(-t)) - p) < 1e-12
    assert _lib.logit_threshold(0.0) == -np.inf and _lib.logit_threshold(1.01) == np.inf
    # p == 1: the float32 sigmoid's saturation point, as the oracle finds it
    t1 = _lib.logit_threshold(1.0)
    assert t1 == float(O.sigmoid_f32_threshold(1.0))
    z = torch.tensor([np.nextafter(np.float32(t1), np.float32(0)), t1], dtype=torch.float32)
    assert (torch.sigmoid(z) >= 1.0).tolist() == [False, True]


# ── native file store (host code: runs without a GPU) ───────────────────────

def _file_store_or_skip(cold_bin, cold_idx, direct, threads):
    from oi2.filestore import FileStore
    try:
        return FileStore(cold_bin, cold_idx, direct=direct, threads=threads)
    except oi2.OI2Error as e:
        if direct and "O_DIRECT" in str(e):
            pytest.skip(f"this file system refuses O_DIRECT: {e}")
        raise


@pytest.mark.parametrize("direct,threads", [(False, 1), (False, 4), (True, 1), (True, 3)],
                         ids=["mmap-1", "mmap-4", "direct-1", "direct-3"])
def test_file_store_reads_records_in_request_order(direct, threads):
    """oi2_file_store_read returns exactly the file's record bytes
    (splitter.py:354-403's per-record slices), in request order with
    duplicates kept, whether read through the mapping or with O_DIRECT page
    reads (records straddling pages, neighbours merged into one read, the
    last record of the file); bad slots and sections are refused."""
    with tempfile.TemporaryDirectory(dir=os.path.dirname(os.path.abspath(__file__))) as tmp:
        cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp, 4, 40, 3)
        raw = np.frombuffer(open(cold_bin, "rb").read(), np.uint8)
        index = np.load(cold_idx)
        fs = _file_store_or_skip(cold_bin, cold_idx, direct, threads)
        try:
            assert fs.sections == 4 and list(fs.n_records) == [40] * 4
            rng = np.random.default_rng(0)
            for li in range(4):
                base = int(index[li, 0, 0]) + 16
                reqs = [np.arange(40), np.arange(40)[::-1], rng.integers(0, 40, 97),
                        np.array([39]), np.array([5, 5, 6, 0, 39, 20])]
                for req in reqs:
                    out = np.full((len(req), 6400), 0xAB, np.uint8)
                    assert fs.read(li, req, out) == len(req)
                    want = np.stack([raw[base + 6400 * s: base + 6400 * (s + 1)] for s in req])
                    assert np.array_equal(out, want)
                assert fs.nids(li).tolist() == layers[li][0]
            pinned_like = torch.empty(3 * 6400, dtype=torch.uint8)
            fs.read(2, [1, 2, 3], pinned_like)
            assert np.array_equal(pinned_like.numpy(), raw[int(index[2, 0, 0]) + 16 + 6400:
                                                           int(index[2, 0, 0]) + 16 + 4 * 6400])
            with pytest.raises(oi2.OI2Error, match="outside section"):
                fs.read(0, [40], np.empty((1, 6400), np.uint8))
            with pytest.raises(oi2.OI2Error, match="section 9 out of range"):
                fs.read(9, [0], np.empty((1, 6400), np.uint8))
            with pytest.raises(ValueError, match="records need"):
                fs.read(0, [0, 1], np.empty((1, 6400), np.uint8))
        finally:
            fs.close()


@pytest.mark.parametrize("gap", [0, 4096, 16384, 131072, 524288])
def test_file_store_direct_read_gap(gap):
    """O_DIRECT reads that merge records across gaps of 0 to 512 KB (whole
    sections in one read at the largest) return the same bytes as the
    file; gaps outside 0 .. 512 KB are refused."""
    from oi2 import _lib
    with tempfile.TemporaryDirectory(dir=os.path.dirname(os.path.abspath(__file__))) as tmp:
        cold_bin, cold_idx, config, layers = synthetic_cold_file(tmp, 2, 200, 5)
        raw = np.frombuffer(open(cold_bin, "rb").read(), np.uint8)
        index = np.load(cold_idx)
        fs = _file_store_or_skip(cold_bin, cold_idx, True, 3)
        try:
            _lib.check(_lib.load_library().oi2_file_store_set_read_gap(fs._h, gap))
            rng = np.random.default_rng(gap)
            for li in range(2):
                base = int(index[li, 0, 0]) + 16
                for req in (rng.choice(200, 30, replace=False), rng.integers(0, 200, 120), np.arange(200)):
                    out = np.empty((len(req), 6400), np.uint8)
                    fs.read(li, req, out)
                    want = np.stack([raw[base + 6400 * s: base + 6400 * (s + 1)] for s in req])
                    assert np.array_equal(out, want)
            for bad in (-1, 524289):
                with pytest.raises(oi2.OI2Error, match="read gap"):
                    _lib.check(_lib.load_library().oi2_file_store_set_read_gap(fs._h, bad))
        finally:
            fs.close()
