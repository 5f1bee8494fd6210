"""Pins the oracle's routing (Int8-gemm/moe_common.cpp:146-216) and block
dots (Int8-gemm/gemm_kernels.cpp:102-133, 262-309) by brute force."""
import numpy as np
import pytest
import torch

import oracle
import nanovllm_moe.formats as fmt


def _brute_route(ids, E):
    T, K = ids.shape
    pairs = [(int(ids[t, k]), t, k) for t in range(T) for k in range(K) if 0 <= ids[t, k] < E]
    order = sorted(range(len(pairs)), key=lambda i: (pairs[i][0], i))  # stable by expert
    return [pairs[i] for i in order]


@pytest.mark.parametrize("T,K,E,seed", [(1, 8, 128, 0), (7, 8, 16, 1), (33, 10, 64, 2), (5, 1, 4, 3), (64, 8, 128, 4)])
def test_route_matches_stable_sort(T, K, E, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-2, E + 2, size=(T, K)).astype(np.int32)   # includes invalid ids
    counts, starts, tmap, scat = oracle.route(ids, E)
    valid = (ids >= 0) & (ids < E)
    assert counts.sum() == valid.sum()
    assert np.array_equal(counts, np.bincount(ids[valid], minlength=E))
    assert starts[0] == 0 and np.array_equal(np.diff(starts), counts)
    brute = _brute_route(ids, E)
    assert [(t, k) for _, t, k in brute] == [tuple(p) for p in tmap]
    for t in range(T):
        for k in range(K):
            if valid[t, k]:
                assert tuple(tmap[scat[t, k]]) == (t, k)
            else:
                assert scat[t, k] == -1


def test_route_topk_restriction():
    ids = np.zeros((2, 3), np.int32)
    with pytest.raises(RuntimeError):
        oracle.route(ids, 8, restrict_topk=True)
    oracle.route(np.zeros((2, 8), np.int32), 8, restrict_topk=True)


def test_q4_nibble_order_known_answer():
    # word 0x76543210 holds nibbles 0..7 at k = 0..7 -> values nibble - 8
    w = np.array([[0x76543210, 0xFEDCBA98, 0, 0]], dtype=np.uint32).view(np.int32)
    a = np.zeros((1, 32), np.int8)
    a[0, 3] = 1      # picks element k=3 -> 3-8 = -5
    a[0, 12] = 2     # k=12 -> nibble 0xC=12 -> 4, times 2 = 8
    a[0, 20] = 7     # k=20 -> word 2 = 0 -> -8, times 7 = -56
    isum = oracle.block_dots(1, a, w, N=1, K=32)
    assert isum[0, 0, 0] == -5 + 8 - 56
    assert np.array_equal(fmt.q4_0_unpack(torch.from_numpy(w))[0, :16].numpy(), np.arange(16) - 8)


@pytest.mark.parametrize("qt", [0, 1])
def test_block_dots_brute_force(qt):
    rng = np.random.default_rng(5 + qt)
    M, N, K = 3, 5, 128
    a = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    if qt == 0:
        w = rng.integers(-128, 128, size=(N, K)).astype(np.int8)
        wv = w.astype(np.int64)
    else:
        w = rng.integers(0, 2**32, size=(N, K // 8), dtype=np.uint64).astype(np.uint32).view(np.int32)
        wv = fmt.q4_0_unpack(torch.from_numpy(w)).numpy()
    isum = oracle.block_dots(qt, a, w, N, K)
    ref = np.einsum("mbi,nbi->mnb", a.astype(np.int64).reshape(M, K // 32, 32), wv.reshape(N, K // 32, 32))
    assert np.array_equal(isum.astype(np.int64), ref)
    # extremes stay exact in int32
    a2 = np.full((1, K), -128, np.int8)
    w2 = np.full((1, K), -128, np.int8) if qt == 0 else np.zeros((1, K // 8), np.int32)
    expect = 32 * 128 * 128 if qt == 0 else 32 * 128 * 8
    assert (oracle.block_dots(qt, a2, w2, 1, K) == expect).all()
