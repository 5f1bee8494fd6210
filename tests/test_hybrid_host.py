"""The host half of the hybrid offload executor (mi_moe_hybrid_host_forward)
against the oracle's fused forwards (Int8-gemm/q8_gemm.cpp:276-646 for Q8_0 /
Q4_0, the W4A16 restatement), on the CPU: handles made with every expert on
the host need no HIP device.  The cold-expert partial must equal the oracle's
fp32 output over the routed pairs of the cold experts only (the others'
ids set to -1) -- bit for bit for Q8_0 / Q4_0, which run on the host engine
of the reference CPU algorithm, within 1e-5 for W4A16 -- and be independent
of the thread count."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
import nanovllm_moe as nm
from nanovllm_moe import HybridMoE
from helpers import bits, max_rel_err, topk_routing, w4a16_random
from test_oracle_forward import _q_weights


def _x(T, H, seed, dt):
    return (torch.randn(T, H, generator=torch.Generator().manual_seed(seed)) * 0.7).to(dt)


def _mask_ids(ids, cold):
    """ids with the pairs of non-cold experts dropped (-1), numpy int32."""
    ids = np.array(ids, dtype=np.int32, copy=True)
    keep = np.isin(ids, np.array(sorted(cold), dtype=np.int32))
    ids[~keep] = -1
    return ids


def _oracle_q(qt, x, ids, tw, ws, E, I):
    acode = 1 if x.dtype == torch.bfloat16 else 0
    scode = 1 if ws[1].dtype == torch.bfloat16 else 0
    _, yf = oracle.moe_forward_q(qt, acode, scode, bits(x), tw, ids, ws[0], bits(ws[1]), ws[2], bits(ws[3]), E, I)
    return yf


def _oracle_w4(x, ids, tw, ws, E, I):
    acode = 1 if x.dtype == torch.bfloat16 else 0
    scode = 1 if ws[2].dtype == torch.bfloat16 else 0
    _, yf = oracle.moe_forward_w4a16(acode, scode, bits(x), tw, ids, ws[0].numpy(), ws[1].numpy(), bits(ws[2]),
                                     ws[3].numpy(), ws[4].numpy(), bits(ws[5]), E, I)
    return yf


def _q_hybrid(qt, E, H, I, cold, ws, threads=2):
    hm = HybridMoE(E, H, I, qt, host_experts=cold, num_threads=threads)
    hm.store_quantized(torch.from_numpy(np.ascontiguousarray(ws[0])), ws[1],
                       torch.from_numpy(np.ascontiguousarray(ws[2])), ws[3])
    return hm


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("adt,sdt", [(torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16)])
def test_q_all_host_matches_oracle(qt, adt, sdt):
    E, H, I, T, K = 8, 256, 128, 7, 8
    ws = _q_weights(qt, E, H, I, 20 + qt, sdt)
    ids, tw = topk_routing(T, E, K, seed=5)
    ids = ids.numpy().copy()
    ids[1, 3] = -1          # dropped id
    ids[4, :] = E + 2       # a token with no valid id -> zero row
    x = _x(T, H, 6, adt)
    hm = _q_hybrid(qt, E, H, I, range(E), ws)
    y = hm.host_forward(x, torch.from_numpy(ids), tw)
    ref = _oracle_q(qt, x, ids, tw.numpy(), ws, E, I)
    # the host engine computes in the oracle's operation order: bit-equal fp32 partial
    assert np.array_equal(y.numpy().view(np.uint32), ref.view(np.uint32))
    assert torch.all(y[4] == 0)
    assert hm.stats()["last_host_pairs"] == int(((ids >= 0) & (ids < E)).sum())


@pytest.mark.parametrize("qt", [0, 1])
def test_q_cold_subset_is_the_masked_forward(qt):
    E, H, I, T, K = 8, 256, 128, 9, 8
    ws = _q_weights(qt, E, H, I, 30 + qt, torch.float16)
    cold = [1, 4, 6]
    ids, tw = topk_routing(T, E, K, seed=7)
    x = _x(T, H, 8, torch.bfloat16)
    hm = _q_hybrid(qt, E, H, I, range(E), ws)   # all on the host, masked routing
    masked = _mask_ids(ids.numpy(), cold)
    y = hm.host_forward(x, torch.from_numpy(masked), tw)
    ref = _oracle_q(qt, x, masked, tw.numpy(), ws, E, I)
    assert np.array_equal(y.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T,K,threads", [(1, 1, 8), (2, 1, 8), (3, 1, 7), (1, 8, 16)])
def test_q_few_tasks_many_threads(qt, T, K, threads):
    """Fewer expert tasks than half the threads: each task's rows are split
    over up to threads/tasks parts of 16-row panels (2 in the reference);
    the partial stays bit-equal to the oracle."""
    E, H, I = 8, 512, 256
    ws = _q_weights(qt, E, H, I, 90 + qt, torch.float16)
    ids, tw = topk_routing(T, E, K, seed=91 + K)
    x = _x(T, H, 92, torch.bfloat16)
    hm = _q_hybrid(qt, E, H, I, range(E), ws, threads=threads)
    y = hm.host_forward(x, ids, tw)
    ref = _oracle_q(qt, x, ids.numpy(), tw.numpy(), ws, E, I)
    assert np.array_equal(y.numpy().view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("adt,sdt", [(torch.bfloat16, torch.bfloat16), (torch.float16, torch.float16)])
@pytest.mark.parametrize("K", [1, 4, 8])
def test_w4a16_all_host_matches_oracle(adt, sdt, K):
    E, H, I, T = 8, 512, 256, 6
    ws = w4a16_random(E, H, I, seed=40 + K, scale_dtype=sdt)
    ids, tw = topk_routing(T, E, K, seed=41)
    ids = ids.numpy().copy()
    ids[0, 0] = -3
    x = _x(T, H, 42, adt)
    hm = HybridMoE(E, H, I, nm.W4A16, host_experts=range(E), num_threads=3)
    hm.store_awq(*ws)
    y = hm.host_forward(x, torch.from_numpy(ids), tw)
    ref = _oracle_w4(x, ids, tw.numpy(), ws, E, I)
    assert max_rel_err(y, torch.from_numpy(ref)) < 1e-5   # fp32, per-group zero fold vs per-element dequant


def test_w4a16_token_blocks_and_thread_count():
    """T above the executor's 256-token pass, cold subset, 1 vs 4 threads bit-identical."""
    E, H, I, T, K = 8, 512, 128, 300, 2
    ws = w4a16_random(E, H, I, seed=50)
    ids, tw = topk_routing(T, E, K, seed=51)
    cold = [0, 3, 7]
    x = _x(T, H, 52, torch.bfloat16)
    masked = torch.from_numpy(_mask_ids(ids.numpy(), cold))
    ys = []
    for threads in (1, 4):
        hm = HybridMoE(E, H, I, nm.W4A16, host_experts=range(E), num_threads=threads)
        hm.store_awq(*ws)
        ys.append(hm.host_forward(x, masked, tw))
    assert torch.equal(ys[0], ys[1])
    ref = _oracle_w4(x, masked.numpy(), tw.numpy(), ws, E, I)
    assert max_rel_err(ys[0], torch.from_numpy(ref)) < 1e-5
    no_cold = ~np.isin(ids.numpy(), cold).any(axis=1)
    assert no_cold.any() and torch.all(ys[0][torch.from_numpy(no_cold)] == 0)


def test_hybrid_host_only_handle_errors():
    L = nm.capi()
    E, H, I = 4, 512, 128
    h = ctypes.c_void_p()
    assert L.mi_moe_hybrid_create(E, H, I, 2, None, 0, ctypes.byref(h)) == 1          # null mask
    mask = (ctypes.c_uint8 * E)(1, 1, 1, 1)
    assert L.mi_moe_hybrid_create(E, 500, I, 2, mask, 0, ctypes.byref(h)) == 1       # H % 512
    assert L.mi_moe_hybrid_create(E, H, I, 2, mask, 999, ctypes.byref(h)) == 1       # threads
    assert L.mi_moe_hybrid_create(E, H, I, 2, mask, 2, ctypes.byref(h)) == 0
    x = np.zeros((2, H), np.uint16)
    ids = np.zeros((2, 1), np.int32)
    w = np.ones((2, 1), np.float32)
    y = np.zeros((2, H), np.float32)
    p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    assert L.mi_moe_hybrid_host_forward(h, p(x), p(w), p(ids), 2, 1, 1, p(y)) == 2   # not loaded
    assert L.mi_moe_hybrid_host_forward(h, p(x), p(w), p(ids), 2, 0, 1, p(y)) in (1, 2)
    dev, host, hb = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
    assert L.mi_moe_hybrid_get_stats(h, ctypes.byref(dev), ctypes.byref(host), ctypes.byref(hb), None, None, None) == 0
    assert (dev.value, host.value, hb.value) == (0, E, 0)
    assert L.mi_moe_hybrid_destroy(h) == 0


def test_hybrid_stats_host_bytes():
    E, H, I = 8, 512, 128
    ws = w4a16_random(E, H, I, seed=60)
    hm = HybridMoE(E, H, I, nm.W4A16, host_experts=range(E), num_threads=1)
    hm.store_awq(*ws)
    st = hm.stats()
    assert st["host_experts"] == E and st["device_experts"] == 0
    assert st["host_weight_bytes"] == sum(t.numel() * t.element_size() for t in ws)


def test_w4a16_task_widths_bit_identical():
    """One cold expert on 1, 4 and 16 threads: the column-block tasks are
    handed out dynamically, and each output column is summed in the same order
    whichever thread takes its block, so the outputs are bit-identical."""
    E, H, I, T, K = 4, 512, 128, 5, 2
    ws = w4a16_random(E, H, I, seed=70)
    ids = torch.tensor([[2, 0], [1, 2], [2, 3], [0, 1], [3, 2]], dtype=torch.int32)
    tw = torch.softmax(torch.randn(T, K, generator=torch.Generator().manual_seed(71)), dim=-1)
    x = _x(T, H, 72, torch.bfloat16)
    masked = torch.from_numpy(_mask_ids(ids.numpy(), [2]))
    ys = []
    for threads in (1, 4, 16):
        hm = HybridMoE(E, H, I, nm.W4A16, host_experts=range(E), num_threads=threads)
        hm.store_awq(*ws)
        ys.append(hm.host_forward(x, masked, tw))
    assert torch.equal(ys[0], ys[1]) and torch.equal(ys[0], ys[2])
    ref = _oracle_w4(x, masked.numpy(), tw.numpy(), ws, E, I)
    assert max_rel_err(ys[0], torch.from_numpy(ref)) < 1e-5
    assert torch.all(ys[0][3] == 0)   # token 3 routes no pair to expert 2


def test_host_forward_rejects_mismatched_shapes():
    """The C ABI trusts T, H and K: HybridMoE checks the tensors first."""
    E, H, I, T, K = 4, 256, 128, 3, 2
    hm = HybridMoE(E, H, I, 0, host_experts=range(E), num_threads=1)
    try:
        x = torch.zeros(T, H, dtype=torch.bfloat16)
        ids = torch.zeros(T, K, dtype=torch.int32)
        w = torch.zeros(T, K, dtype=torch.float32)
        bad = [
            (torch.zeros(T, H + 32, dtype=torch.bfloat16), ids, w),     # hidden size
            (x, torch.zeros(T + 1, K, dtype=torch.int32), w),          # ids rows
            (x, ids, torch.zeros(T - 1, K)),                           # weight rows
            (x, ids, torch.zeros(T, K + 1)),                           # top_k disagree
            (x.reshape(-1), ids, w),                                   # not 2-D
            (x.float(), ids, w),                                       # dtype
        ]
        for args in bad:
            with pytest.raises(ValueError):
                hm.host_forward(*args)
        with pytest.raises(ValueError):   # forward needs HIP tensors, checked first
            hm.forward(x, ids, w)
    finally:
        hm.close()
