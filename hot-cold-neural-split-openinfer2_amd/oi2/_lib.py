"""ctypes binding of liboi2.so (the C ABI declared in include/oi2.h).

The library is the only compute path: if it has not been built, or no
gfx950 device is present, calls raise instead of falling back to anything.
"""
from __future__ import annotations

import ctypes
import math
import os
from ctypes import POINTER, Structure, c_float, c_int32, c_size_t, c_void_p

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liboi2.so")

OI2_OK = 0
OI2_EUNSUPPORTED = 4
ACT_SILU, ACT_RELU = 0, 1
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
ABI_VERSION = 2
HIDDEN = 4096
SEL_CHUNK = 256


class OI2Error(RuntimeError):
    pass


class Hot(Structure):
    _fields_ = [("n_hot", c_int32), ("down_stride", c_int32), ("gate_q", c_void_p),
                ("up_q", c_void_p), ("down_q", c_void_p), ("gate_scale", c_void_p),
                ("up_scale", c_void_p), ("down_scale", c_void_p), ("gate_bias", c_void_p)]


class Cold(Structure):
    _fields_ = [("records", c_void_p), ("n_records", c_int32), ("gate_bias", c_void_p)]


class Active(Structure):
    _fields_ = [("slots", c_void_p), ("counts", c_void_p), ("n_chunks", c_int32),
                ("chunk", c_int32), ("expected", c_int32)]


class Predictor(Structure):
    _fields_ = [("inter", c_int32), ("rank", c_int32), ("dtype", c_int32), ("down_w", c_void_p),
                ("up_w", c_void_p), ("up_b", c_void_p)]


class Attn(Structure):
    _fields_ = [("n_q", c_int32), ("n_kv", c_int32), ("wq", c_void_p), ("wk", c_void_p),
                ("wv", c_void_p), ("wo", c_void_p), ("norm_w", c_void_p)]


class Layer(Structure):
    _fields_ = [("hot", Hot), ("cold", Cold), ("lut", c_void_p), ("norm_w", c_void_p),
                ("pred", Predictor)]


_SIGS = {
    "oi2_last_error": (ctypes.c_char_p, []),
    "oi2_abi_version": (c_int32, []),
    "oi2_record_bytes": (c_int32, []),
    "oi2_dequant_records": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p,
                                      c_void_p, c_void_p]),
    "oi2_rmsnorm": (c_int32, [c_void_p, c_void_p, c_int32, c_float, c_void_p, c_void_p]),
    "oi2_ffn_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "oi2_ffn_forward": (c_int32, [c_void_p, c_int32, c_void_p, c_float, POINTER(Hot), POINTER(Cold),
                                  POINTER(Active), c_int32, c_int32, c_int32, c_void_p, c_void_p,
                                  c_void_p, c_size_t, c_void_p]),
    "oi2_ffn_forward_chain": (c_int32, [c_void_p, c_int32, c_void_p, c_float, c_void_p, POINTER(Hot),
                                        POINTER(Cold), POINTER(Active), c_int32, c_int32, c_int32,
                                        c_void_p, c_void_p, c_void_p, c_float, c_void_p, c_void_p,
                                        c_size_t, c_void_p]),
    "oi2_sparse_ffn_dense_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "oi2_sparse_ffn_dense": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32,
                                       c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                       c_void_p]),
    "oi2_ffn_forward_noalloc": (c_int32, [c_void_p, c_int32, c_void_p, c_float, POINTER(Hot),
                                          POINTER(Cold), POINTER(Active), c_int32, c_int32, c_int32,
                                          c_void_p, c_void_p, c_void_p]),
    "oi2_ffn_noalloc_scratch_bytes": (c_size_t, []),
    "oi2_ffn_noalloc_max_expected": (c_int32, []),
    "oi2_predict_workspace_bytes": (c_size_t, [POINTER(Predictor)]),
    "oi2_predict": (c_int32, [c_void_p, c_int32, c_int32, POINTER(Predictor), c_float, c_void_p,
                              c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "oi2_predict_select": (c_int32, [c_void_p, c_int32, c_void_p, c_float, POINTER(Predictor),
                                     c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "oi2_stack_create": (c_int32, [POINTER(Layer), c_int32, c_int32, c_float, c_int32, c_int32,
                                   c_float, POINTER(c_void_p)]),
    "oi2_stack_decode": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p]),
    "oi2_stack_predict": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p]),
    "oi2_stack_layer": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p]),
    "oi2_stack_set_graph": (c_int32, [c_void_p, c_int32]),
    "oi2_stack_set_expected_active": (c_int32, [c_void_p, c_int32]),
    "oi2_stack_profile": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, POINTER(c_float),
                                    POINTER(c_float), c_void_p]),
    "oi2_stack_set_staging": (c_int32, [c_void_p, c_int32]),
    "oi2_stack_profile_staging": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, POINTER(c_float),
                                            c_void_p]),
    "oi2_stack_trace": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "oi2_stack_selection_layout": (c_int32, [c_void_p, POINTER(c_int32), POINTER(c_int32)]),
    "oi2_stack_set_token_kernel": (c_int32, [c_void_p, c_int32]),
    "oi2_stack_token_kernel": (c_int32, [c_void_p]),
    "oi2_stack_status": (c_int32, [c_void_p, c_void_p]),
    "oi2_stack_set_wait_bound": (c_int32, [c_void_p, c_int32]),
    "oi2_stack_profile_token": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, POINTER(c_float),
                                          c_void_p]),
    "oi2_stack_trace_token": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_void_p]),
    "oi2_stack_destroy": (c_int32, [c_void_p]),
    "oi2_file_store_open": (c_int32, [ctypes.c_char_p, c_void_p, c_int32, c_int32, c_int32,
                                      POINTER(c_void_p)]),
    "oi2_file_store_read": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_void_p]),
    "oi2_file_store_stage": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_void_p, c_void_p,
                                       c_void_p]),
    "oi2_file_store_set_read_gap": (c_int32, [c_void_p, ctypes.c_int64]),
    "oi2_file_store_close": (c_int32, [c_void_p]),
    "oi2_attn_workspace_bytes": (c_size_t, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "oi2_attn_forward": (c_int32, [c_void_p, c_int32, c_int32, POINTER(Attn), c_float, c_void_p,
                                   c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                   c_void_p, c_void_p, c_size_t, c_void_p]),
    "oi2_section_bytes": (c_size_t, [c_int32]),
    "oi2_quantize_section": (c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                       c_void_p]),
}

_lib = None


def load_library():
    """Load liboi2.so and declare every exported signature (no GPU needed)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise OI2Error(f"{LIB_PATH} is missing: build it with `python -c 'import "
                           f"__graft_entry__ as g; g.build()'` (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.oi2_abi_version() != ABI_VERSION:
            raise OI2Error("liboi2.so ABI version mismatch")
        _lib = lib
    return _lib


def lib():
    """The library, for compute calls: also requires a visible GPU."""
    L = load_library()
    if not torch.cuda.is_available():
        raise OI2Error("oi2 kernels need a gfx950 GPU; none is visible")
    return L


def check(rc: int):
    if rc != OI2_OK:
        msg = load_library().oi2_last_error().decode(errors="replace")
        raise OI2Error(f"oi2 call failed ({rc}): {msg}")


def ptr(t) -> int | None:
    if t is None:
        return None
    return t.data_ptr()


def dtype_code(dtype) -> int:
    """The ABI's dtype code of a torch floating dtype (fp16, fp32, bf16)."""
    codes = {torch.float16: DTYPE_F16, torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16}
    if dtype not in codes:
        raise TypeError(f"dtype {dtype} is not float16, float32 or bfloat16")
    return codes[dtype]


def stream_handle(device=None) -> int | None:
    s = torch.cuda.current_stream(device).cuda_stream
    return s or None


def logit_threshold(p: float) -> float:
    """The logit cut the kernels apply for predict_mask's ``sigmoid(l) >= p``
    (predictor.py:77-79): l >= log(p / (1 - p)) for 0 < p < 1.  At the edges
    the reference's float32 sigmoid decides: p <= 0 passes every logit, p == 1
    passes the logits whose float32 sigmoid rounds to 1.0 (l >= 16.6355...),
    and p > 1 passes none."""
    if p <= 0.0:
        return -math.inf
    if p > 1.0:
        return math.inf
    if p == 1.0:
        return _sigmoid_f32_cut(1.0)
    return math.log(p / (1.0 - p))


def _sigmoid_f32_cut(p: float) -> float:
    """Smallest float32 l with torch.sigmoid(l) >= p in float32, by bisection
    over the ordered float32 bit patterns."""
    def key_to_f(k):
        u = (k ^ 0xFFFFFFFF) if not k >> 31 else (k & 0x7FFFFFFF)
        return torch.tensor([u], dtype=torch.int64).to(torch.int32).view(torch.float32)

    def passes(k):
        return bool(torch.sigmoid(key_to_f(k))[0] >= p)

    lo, hi = 0x007FFFFF, 0xFF800000           # keys of -inf and +inf
    if passes(lo):
        return -math.inf
    if not passes(hi - 1):
        return math.inf
    while hi - lo > 1:
        mid = (lo + hi) // 2
        if passes(mid):
            hi = mid
        else:
            lo = mid
    return float(key_to_f(hi)[0])
