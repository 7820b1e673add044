"""Helpers for the GPU parity tests: device layouts -> oracle inputs."""
import numpy as np
import torch

from oracle import oracle as O

EPS = 1e-5


def hot_dense(hot):
    if hot is None or hot.n_hot == 0:
        return None, None, None
    return O.hot_to_dense(hot.gate_q.cpu().numpy(), hot.up_q.cpu().numpy(),
                          hot.down_q[:, :hot.n_hot].cpu().numpy(), hot.gate_scale.cpu().numpy(),
                          hot.up_scale.cpu().numpy(), hot.down_scale.cpu().numpy())


def cold_dense(records, slots):
    recs = records.cpu().numpy() if torch.is_tensor(records) else records
    s = slots.cpu().numpy() if torch.is_tensor(slots) else np.asarray(slots)
    return O.records_to_dense(recs, s)


def normed_f16(x, norm_w, eps=EPS):
    """RMSNorm in float64 rounded to fp16 (the activation dtype of the
    normalised hidden state), returned as float64 values."""
    xv = x.float().cpu().numpy()
    if norm_w is None:
        return xv.astype(np.float16).astype(np.float64)
    return O.rmsnorm(xv, norm_w.float().cpu().numpy(), eps).astype(np.float16).astype(np.float64)


def assert_ffn_close(y, ref, tol=1e-2, cos_min=0.9999, what="ffn"):
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    assert np.isfinite(y).all(), f"{what}: non-finite output"
    err, cos = O.rel_err(y, ref), O.cosine(y, ref)
    assert err <= tol and cos >= cos_min, f"{what}: max rel err {err:.3e}, cosine {cos:.7f}"
    return err, cos


def chunked_ids(counts, ids, chunk=256):
    c = counts.cpu().tolist()
    row = ids.cpu()
    out = []
    for k, n in enumerate(c):
        out.extend(row[k * chunk: k * chunk + n].tolist())
    return out


def pred_weights(p):
    return (p.down_w.float().cpu().numpy().astype(np.float64),
            p.up_w.float().cpu().numpy().astype(np.float64),
            p.up_b.float().cpu().numpy().astype(np.float64))


def query_for(xn_rows_f16, dtype):
    """engine.py:277 + predictor.py:455: batch mean (fp16) cast to the
    predictor dtype."""
    q = O.query(xn_rows_f16).astype(np.float32)
    if dtype == torch.bfloat16:
        q = O.to_bf16(q)
    return q.astype(np.float64)
