"""CPU oracle for the fused-MoE hot path -- TEST INFRASTRUCTURE ONLY.

This package is the *checker*: a plain-C restatement of the reference CPU
fused-MoE algorithm (Int8-gemm/q8_gemm.cpp:276-646 and the kernels it calls)
plus an fp32 W4A16 restatement.  Only ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg may import it; the product path
(``moe-ascend-opt_amd``) never does.

Parity status per function (how each is pinned; see tests/test_oracle_*.py):
  quantize_block_q8_0 / quantize_act_q8_0 / quantize_weight_q8_0
      closed-form cases (zero block, +-amax -> +-127, exact multiples, RNE
      ties), the round-to-nearest error bound, golden fixtures.
  route                 invariants + numpy stable-argsort brute force.
  block_dots            numpy int64 brute force (exact).
  silu_and_mul / expf   libm/numpy within 2 ulp, special values.
  moe_forward_q         dense float64 torch formula over dequantized weights
                        (tight) and the reference's own fp16 dense check
                        (Int8-gemm/test/fused_moe_cpu.py:40-95, loose).
  awq_dequant           known-answer packed words + pack/unpack round trip.
  moe_forward_w4a16     dense float64 torch formula over dequantized weights.
  topk_softmax          the reference's own formula (torch.topk + torch.softmax,
                        Int8-gemm/test/fused_moe_cpu.py:20-37): ids exact, weights
                        within a few ulp; ties, K = E, -inf logits, float64 softmax.
The exact fp32 bits of the ARM build (``-ffast-math``, ggml's exp polynomial)
are not reproducible off-ARM: those bits are "parity unpinned" and are
compared at tolerance.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liborc.so")
_lib = None

F16, BF16 = 0, 1
Q8_0, Q4_0, W4A16 = 0, 1, 2


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc only)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.orc_expf.restype = ctypes.c_float
        _lib.orc_expf.argtypes = [ctypes.c_float]
        _lib.orc_route.restype = ctypes.c_int64
        _lib.orc_moe_forward_q.restype = ctypes.c_int
        _lib.orc_moe_forward_w4a16.restype = ctypes.c_int
        for fn in ("orc_f32_to_f16", "orc_f32_to_bf16"):
            getattr(_lib, fn).restype = ctypes.c_uint16
            getattr(_lib, fn).argtypes = [ctypes.c_float]
        for fn in ("orc_f16_to_f32", "orc_bf16_to_f32"):
            getattr(_lib, fn).restype = ctypes.c_float
            getattr(_lib, fn).argtypes = [ctypes.c_uint16]
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _i64(v):
    return ctypes.c_int64(int(v))


# ---------------------------------------------------------------- scalars
def expf(x: float) -> float:
    return float(lib().orc_expf(ctypes.c_float(x)))


def expf_vec(x: np.ndarray) -> np.ndarray:
    f = lib().orc_expf
    return np.array([f(ctypes.c_float(float(v))) for v in x.ravel()],
                    dtype=np.float32).reshape(x.shape)


# ---------------------------------------------------------------- quant
def quantize_block_q8_0(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == 32
    d = np.zeros(1, np.float32)
    qs = np.zeros(32, np.int8)
    lib().orc_quantize_block_q8_0(_p(x), _p(d), _p(qs))
    return float(d[0]), qs


def quantize_act_q8_0(x_bits: np.ndarray, act_dtype: int):
    """x_bits: uint16 [T,H] raw fp16/bf16 -> (qs int8 [T,H], d f32 [T,H/32])."""
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x_bits.shape
    qs = np.zeros((T, H), np.int8)
    d = np.zeros((T, H // 32), np.float32)
    lib().orc_quantize_act_q8_0(_p(x_bits), ctypes.c_int(act_dtype), _i64(T), _i64(H), _p(qs), _p(d))
    return qs, d


def quantize_weight_q8_0(w: np.ndarray):
    """w f32 [N,K] -> (qs int8 [N,K], d fp16-bits uint16 [N,K/32])."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    qs = np.zeros((N, K), np.int8)
    d = np.zeros((N, K // 32), np.uint16)
    lib().orc_quantize_weight_q8_0(_p(w), _i64(N), _i64(K), _p(qs), _p(d))
    return qs, d


# ---------------------------------------------------------------- routing
def route(ids: np.ndarray, E: int, restrict_topk: bool = False):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, K = ids.shape
    counts = np.zeros(E, np.int32)
    starts = np.zeros(E + 1, np.int32)
    tmap = np.zeros(2 * T * K + 2, np.int32)
    scat = np.zeros(T * K + 1, np.int32)
    n = lib().orc_route(_p(ids), _i64(T), _i64(K), _i64(E), _p(counts), _p(starts),
                        _p(tmap), _p(scat), ctypes.c_int(1 if restrict_topk else 0))
    if n < 0:
        raise RuntimeError("Unsupported top_k. Only 1,8,10 are supported.")
    return counts, starts, tmap[: 2 * n].reshape(n, 2), scat[: T * K].reshape(T, K)


# ---------------------------------------------------------------- block dots
def block_dots(qt: int, a_qs: np.ndarray, w_qs: np.ndarray, N: int, K: int):
    a_qs = np.ascontiguousarray(a_qs, dtype=np.int8)
    M = a_qs.shape[0]
    w_qs = np.ascontiguousarray(w_qs)
    out = np.zeros((M, N, K // 32), np.int32)
    lib().orc_block_dots(ctypes.c_int(qt), _p(a_qs), _i64(M), _p(w_qs), _i64(N), _i64(K), _p(out))
    return out


def silu_and_mul(row: np.ndarray) -> np.ndarray:
    row = np.array(row, dtype=np.float32, copy=True)
    ish = row.size // 2
    lib().orc_silu_and_mul(_p(row), _i64(ish))
    return row[:ish].copy()


# ---------------------------------------------------------------- forward
def moe_forward_q(qt, act_dtype, scale_dtype, x_bits, topk_w, topk_ids,
                  gate_up_qs, gate_up_d, down_qs, down_d, E, I, tp=1):
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x_bits.shape
    K = topk_ids.shape[1]
    y = np.zeros((T, H), np.uint16)
    yf = np.zeros((T, H), np.float32)
    topk_w = np.ascontiguousarray(topk_w, dtype=np.float32)
    topk_ids = np.ascontiguousarray(topk_ids, dtype=np.int32)
    rc = lib().orc_moe_forward_q(
        ctypes.c_int(qt), ctypes.c_int(act_dtype), ctypes.c_int(scale_dtype),
        _p(x_bits), _p(y), _p(yf), _p(topk_w), _p(topk_ids),
        _p(np.ascontiguousarray(gate_up_qs)), _p(np.ascontiguousarray(gate_up_d, dtype=np.uint16)),
        _p(np.ascontiguousarray(down_qs)), _p(np.ascontiguousarray(down_d, dtype=np.uint16)),
        _i64(T), _i64(H), _i64(E), _i64(I), _i64(tp), _i64(K))
    if rc != 0:
        raise RuntimeError("orc_moe_forward_q failed (unsupported top_k or shape)")
    return y, yf


def awq_dequant(qweight, qzeros, scales_bits, scale_dtype, group):
    qweight = np.ascontiguousarray(qweight, dtype=np.int32)
    K, N8 = qweight.shape
    N = N8 * 8
    w = np.zeros((N, K), np.float32)
    lib().orc_awq_dequant(_p(qweight), _p(np.ascontiguousarray(qzeros, dtype=np.int32)),
                          _p(np.ascontiguousarray(scales_bits, dtype=np.uint16)),
                          ctypes.c_int(scale_dtype), _i64(K), _i64(N), _i64(group), _p(w))
    return w


def topk_softmax(logits: np.ndarray, K: int, renormalize: bool = True):
    """Router top-k + softmax (make_topk_from_logits_cpu,
    Int8-gemm/test/fused_moe_cpu.py:20-37): logits [T, E] float32 ->
    (ids [T, K] int32, w [T, K] float32); equal logits: lower id first."""
    x = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = x.shape
    ids = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float32)
    rc = lib().orc_topk_softmax(_p(x), _i64(T), _i64(E), _i64(K), ctypes.c_int(1 if renormalize else 0),
                                _p(ids), _p(w))
    if rc != 0:
        raise ValueError("orc_topk_softmax: bad sizes")
    return ids, w


def moe_forward_w4a16(act_dtype, scale_dtype, x_bits, topk_w, topk_ids,
                      w13_q, w13_z, w13_s, w2_q, w2_z, w2_s, E, I, group=128,
                      nthreads=1):
    x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
    T, H = x_bits.shape
    K = topk_ids.shape[1]
    y = np.zeros((T, H), np.uint16)
    yf = np.zeros((T, H), np.float32)
    rc = lib().orc_moe_forward_w4a16(
        ctypes.c_int(act_dtype), ctypes.c_int(scale_dtype), _p(x_bits), _p(y), _p(yf),
        _p(np.ascontiguousarray(topk_w, dtype=np.float32)),
        _p(np.ascontiguousarray(topk_ids, dtype=np.int32)),
        _p(np.ascontiguousarray(w13_q, dtype=np.int32)), _p(np.ascontiguousarray(w13_z, dtype=np.int32)),
        _p(np.ascontiguousarray(w13_s, dtype=np.uint16)),
        _p(np.ascontiguousarray(w2_q, dtype=np.int32)), _p(np.ascontiguousarray(w2_z, dtype=np.int32)),
        _p(np.ascontiguousarray(w2_s, dtype=np.uint16)),
        _i64(T), _i64(H), _i64(E), _i64(I), _i64(K), _i64(group), ctypes.c_int(nthreads))
    if rc != 0:
        raise RuntimeError("orc_moe_forward_w4a16 failed (shape)")
    return y, yf
