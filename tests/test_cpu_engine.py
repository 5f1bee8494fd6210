"""The host engine of the Q8_0 / Q4_0 layer (mi_moe_cpu_*, the reference CPU
algorithm of Int8-gemm/q8_gemm.cpp:276-646 on x86 cores) against the oracle,
on the CPU.

The engine computes every output in the oracle's operation order (exact int32
block dots, ((float)isum * dw) * da in block order, the same Q8_0 rounding, the
same exp in SiLU, combine in k order, tp partials in shard order, RNE cast),
so the outputs are compared bit for bit -- for every instruction set the host
supports (AVX-512 VNNI, AVX-VNNI, AVX2, scalar), thread counts 1 and 4, tp 1
and 2, the 2-thread-per-task path (few tasks) and the task-per-thread path,
and ragged tasks of 32 + 32 + 5 rows of one expert."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import nanovllm_moe as nm
from helpers import bits, from_bits, topk_routing
from test_oracle_forward import _q_weights


def _engine(qt, E, H, I, ws, threads, tp, sdt):
    L = nm.capi()
    c = ctypes.c_void_p()
    nm.check(L.mi_moe_cpu_create(E, H, I, qt, threads, tp, ctypes.byref(c)), "cpu_create")
    a, b, cq, d = [np.ascontiguousarray(t) if isinstance(t, np.ndarray) else t.contiguous() for t in ws]
    keep = (a, b, cq, d)
    ptr = lambda t: t.ctypes.data if isinstance(t, np.ndarray) else t.data_ptr()
    nm.check(L.mi_moe_cpu_store_quantized(c, ptr(a), ptr(b), ptr(cq), ptr(d), 1 if sdt == torch.bfloat16 else 0),
             "cpu_store")
    return L, c, keep


def _forward(L, c, x, ids, tw):
    y = torch.empty_like(x)
    nm.check(L.mi_moe_cpu_forward(c, x.data_ptr(), y.data_ptr(), tw.data_ptr(), ids.data_ptr(), x.shape[0],
                                  ids.shape[1], nm.dtype_code(x.dtype)), "cpu_forward")
    return y


def _oracle(qt, x, ids, tw, ws, E, I, tp):
    acode = 1 if x.dtype == torch.bfloat16 else 0
    scode = 1 if ws[1].dtype == torch.bfloat16 else 0
    y, _ = oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids.numpy(),
                                np.asarray(ws[0]), bits(ws[1]), np.asarray(ws[2]), bits(ws[3]), E, I, tp=tp)
    return y


def _isas(L, c):
    out = []
    for isa in range(4):
        if L.mi_moe_cpu_set_isa(c, isa) == 0:
            out.append(isa)
    return out


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T,K,threads,tp", [(1, 8, 16, 1), (3, 8, 4, 1), (40, 8, 4, 1), (71, 1, 4, 2),
                                            (5, 10, 1, 2), (2, 8, 8, 2)])
def test_engine_bit_exact_vs_oracle(qt, T, K, threads, tp):
    E, H, I = 12, 256, 128
    sdt = torch.float16 if (T + qt) % 2 else torch.bfloat16
    adt = torch.bfloat16 if T % 3 else torch.float16
    ws = _q_weights(qt, E, H, I, 40 + qt, sdt)
    ids, tw = topk_routing(T, E, K, seed=T * 7 + K)
    ids = ids.clone()
    if T >= 71:
        ids[:, 0] = 5             # one expert with 69 rows: tasks of 32 + 32 + 5
    if T >= 3:
        ids[1, 0] = -1            # dropped
        ids[2, :] = E + 4         # no valid id -> zeros
    x = (torch.randn(T, H, generator=torch.Generator().manual_seed(T)) * 0.8).to(adt)
    L, c, _keep = _engine(qt, E, H, I, ws, threads, tp, sdt)
    try:
        threads_used = ctypes.c_int()
        tp_used = ctypes.c_int()
        nm.check(L.mi_moe_cpu_get_info(c, ctypes.byref(threads_used), ctypes.byref(tp_used), None, None, None,
                                       None), "info")
        assert tp_used.value == tp
        ref = _oracle(qt, x, ids, tw, ws, E, I, tp)
        for isa in _isas(L, c):
            nm.check(L.mi_moe_cpu_set_isa(c, isa), "set_isa")
            y = _forward(L, c, x, ids, tw)
            assert np.array_equal(bits(y), ref), (isa, L.mi_moe_cpu_isa_name(isa))
        if T >= 3:
            assert torch.all(y[2] == 0)
    finally:
        L.mi_moe_cpu_destroy(c)


@pytest.mark.parametrize("tp,per", [(2, 2), (2, 0), (3, 1), (0, 0)])
def test_numa_layout_engine(tp, per):
    """mi_moe_cpu_create_numa: the reference's layout (tp shards, one per NUMA
    node, per threads each); on a host with fewer nodes the affinity CPUs are
    split into tp groups.  The shards sum in shard order, bit-equal to the
    oracle at that tp."""
    import os
    E, H, I, T, K, qt = 12, 256, 192, 6, 8, 0
    ws = _q_weights(qt, E, H, I, 61, torch.float16)
    L = nm.capi()
    c = ctypes.c_void_p()
    nm.check(L.mi_moe_cpu_create_numa(E, H, I, qt, tp, per, ctypes.byref(c)), "cpu_create_numa")
    try:
        a, b, cq, d = [np.ascontiguousarray(t) if isinstance(t, np.ndarray) else t.contiguous() for t in ws]
        ptr = lambda t: t.ctypes.data if isinstance(t, np.ndarray) else t.data_ptr()
        nm.check(L.mi_moe_cpu_store_quantized(c, ptr(a), ptr(b), ptr(cq), ptr(d), 0), "cpu_store")
        thr, tpu, nodes = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        nm.check(L.mi_moe_cpu_get_info(c, ctypes.byref(thr), ctypes.byref(tpu), None, None, ctypes.byref(nodes),
                                       None), "info")
        want_tp = tp if tp > 0 else max(1, nodes.value)
        assert tpu.value == want_tp
        cpus = len(os.sched_getaffinity(0))
        if per > 0 and cpus >= want_tp * per:
            assert thr.value == want_tp * per
        ids, tw = topk_routing(T, E, K, seed=62)
        x = (torch.randn(T, H, generator=torch.Generator().manual_seed(63)) * 0.8).to(torch.bfloat16)
        y = _forward(L, c, x, ids, tw)
        assert np.array_equal(bits(y), _oracle(qt, x, ids, tw, ws, E, I, want_tp))
    finally:
        L.mi_moe_cpu_destroy(c)


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("adt", [torch.bfloat16, torch.float16])
def test_engine_special_values_bit_exact(qt, adt):
    """Hidden rows with NaN, +-inf, signed zeros, subnormals, a zero block and
    values at the dtype's range, and gate_up outputs far beyond exp's range
    (weight scales x 2000, so SiLU sees |gate| in the hundreds): every
    instruction set's Stage A and SiLU + Q8_0 of the intermediate give the
    oracle's bits (NaN compared as NaN)."""
    E, H, I, T, K = 10, 256, 128, 6, 8
    gu_qs, gu_d, dn_qs, dn_d = _q_weights(qt, E, H, I, 70 + qt, torch.float16)
    gu_d = (gu_d.float() * 2000).to(torch.float16)
    ws = (gu_qs, gu_d, dn_qs, dn_d)
    ids, tw = topk_routing(T, E, K, seed=71)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(72)).to(adt)
    big = torch.finfo(adt).max
    tiny = torch.finfo(adt).smallest_normal / 4          # a subnormal of the dtype
    x[1, 5] = float("nan")
    x[1, 40] = float("nan")
    x[2, 64] = float("inf")
    x[2, 200] = -float("inf")
    x[3, :32] = 0.0                                     # a zero block: d = 0
    x[3, 32:64] = -0.0
    x[3, 64:96] = tiny
    x[3, 100] = -tiny
    x[4, ::7] = big
    x[4, 3::11] = -big
    x[5, 128:160] = torch.linspace(-3, 3, 32).to(adt) * 1e-3
    L, c, _keep = _engine(qt, E, H, I, ws, 4, 1, torch.float16)
    try:
        ref = _oracle(qt, x, ids, tw, ws, E, I, 1)
        ref_nan = np.isnan(from_bits(ref, adt).float().numpy())
        for isa in _isas(L, c):
            nm.check(L.mi_moe_cpu_set_isa(c, isa), "set_isa")
            y = _forward(L, c, x, ids, tw)
            y_nan = torch.isnan(y.float()).numpy()
            assert np.array_equal(y_nan, ref_nan), L.mi_moe_cpu_isa_name(isa)
            assert np.array_equal(bits(y)[~y_nan], ref[~ref_nan]), L.mi_moe_cpu_isa_name(isa)
    finally:
        L.mi_moe_cpu_destroy(c)


def test_engine_online_quant_matches_wire_store():
    """quantize_and_store_expert on host (fp32 / fp16 / bf16 weights) gives the
    bytes of the oracle's quantize_weight_only restatement: the same layer
    output as storing the oracle-quantized wire tensors."""
    E, H, I, T, K = 4, 128, 64, 5, 1
    L = nm.capi()
    g = torch.Generator().manual_seed(9)
    w13 = torch.randn(E, 2 * I, H, generator=g) * 0.05
    w2 = torch.randn(E, H, I, generator=g) * 0.05
    c = ctypes.c_void_p()
    nm.check(L.mi_moe_cpu_create(E, H, I, 0, 2, 1, ctypes.byref(c)), "create")
    keep = []
    try:
        for e in range(E):
            for proj, w, dt in ((0, w13[e, :I], torch.float32), (1, w13[e, I:], torch.float16),
                                (2, w2[e], torch.float32)):
                t = w.contiguous().to(dt)
                keep.append(t)
                code = 2 if dt == torch.float32 else (1 if dt == torch.bfloat16 else 0)
                nm.check(L.mi_moe_cpu_quantize_and_store_expert(c, e, proj, t.data_ptr(), code), "quant")
        ids, tw = topk_routing(T, E, K, seed=1)
        x = torch.randn(T, H, generator=g).to(torch.bfloat16)
        y = _forward(L, c, x, ids, tw)
        w13_used = torch.cat([w13[:, :I], w13[:, I:].to(torch.float16).float()], dim=1)
        q13, d13 = oracle.quantize_weight_q8_0(w13_used.reshape(-1, H).numpy())
        q2, d2 = oracle.quantize_weight_q8_0(w2.reshape(-1, I).numpy())
        ws = (q13.reshape(E, 2 * I, H), torch.from_numpy(d13.view(np.float16)).reshape(E, 2 * I, H // 32),
              q2.reshape(E, H, I), torch.from_numpy(d2.view(np.float16)).reshape(E, H, I // 32))
        assert np.array_equal(bits(y), _oracle(0, x, ids, tw, ws, E, I, 1))
    finally:
        L.mi_moe_cpu_destroy(c)


def test_engine_argument_errors():
    L = nm.capi()
    c = ctypes.c_void_p()
    assert L.mi_moe_cpu_create(4, 128, 64, 2, 1, 1, ctypes.byref(c)) == 3        # W4A16: not this engine
    assert L.mi_moe_cpu_create(4, 100, 64, 0, 1, 1, ctypes.byref(c)) == 1        # H % 32
    assert L.mi_moe_cpu_create(4, 128, 96, 0, 1, 2, ctypes.byref(c)) == 1        # I / tp % 32
    assert b"shards" in L.mi_moe_last_error()
    nm.check(L.mi_moe_cpu_create(4, 128, 64, 1, 1, 1, ctypes.byref(c)), "create")
    try:
        assert L.mi_moe_cpu_forward(c, None, None, None, None, 1, 8, 1) == 2      # not loaded
        w = torch.zeros(64, 128)
        assert L.mi_moe_cpu_quantize_and_store_expert(c, 0, 0, w.data_ptr(), 2) == 1   # Q4_0: no online quant
        assert b"store_quantized_repack" in L.mi_moe_last_error()
        assert L.mi_moe_cpu_set_isa(c, 7) == 3
    finally:
        L.mi_moe_cpu_destroy(c)
