"""Oracle router top-k + softmax (make_topk_from_logits_cpu,
Int8-gemm/test/fused_moe_cpu.py:20-37) pinned against the reference's own
formula, torch.topk(largest, sorted) + torch.softmax, and against float64
closed forms; plus the tie rule and edge cases the formula leaves open."""
import numpy as np
import pytest
import torch

import oracle


def _reference(logits, K, renormalize):
    """The reference harness function, restated with torch on the CPU."""
    x = torch.from_numpy(logits)
    val, ids = torch.topk(x, k=K, dim=-1, largest=True, sorted=True)
    if renormalize:
        w = torch.softmax(val, dim=-1)
    else:
        w = torch.gather(torch.softmax(x, dim=-1), -1, ids)
    return ids.to(torch.int32).numpy(), w.to(torch.float32).numpy()


@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("T,E,K,seed", [(1, 128, 8, 0), (8, 128, 8, 1), (64, 256, 8, 2),
                                        (33, 64, 10, 3), (5, 512, 1, 4), (7, 16, 16, 5)])
def test_matches_torch_reference(T, E, K, seed, renorm):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E)).astype(np.float32) * 3
    ids, w = oracle.topk_softmax(logits, K, renorm)
    rid, rw = _reference(logits, K, renorm)
    assert np.array_equal(ids, rid)
    np.testing.assert_allclose(w, rw, rtol=2e-6, atol=1e-7)
    # float64 closed form of the same selection
    v = np.take_along_axis(logits.astype(np.float64), ids.astype(np.int64), 1)
    if renorm:
        ref64 = np.exp(v - v[:, :1]) / np.exp(v - v[:, :1]).sum(1, keepdims=True)
        np.testing.assert_allclose(w.sum(1), 1.0, rtol=1e-6)
    else:
        x64 = logits.astype(np.float64)
        ref64 = np.exp(v - x64.max(1, keepdims=True)) / np.exp(x64 - x64.max(1, keepdims=True)).sum(1, keepdims=True)
    np.testing.assert_allclose(w, ref64, rtol=2e-6, atol=1e-8)
    assert np.all(np.diff(v, axis=1) <= 0)          # descending


def test_ties_lower_id_first_and_edges():
    logits = np.zeros((3, 8), np.float32)
    logits[0] = [1, 5, 5, 0, 5, -1, 2, 5]          # four-way tie at the top
    logits[1] = -np.inf
    logits[1, 6] = 0.0                              # one finite logit, rest -inf
    logits[2] = np.arange(8, dtype=np.float32)      # K = E: full descending order
    ids, w = oracle.topk_softmax(logits[:1], 5, True)
    assert ids.tolist() == [[1, 2, 4, 7, 6]]
    np.testing.assert_allclose(w[0, :4], w[0, 0])   # equal logits, equal weights
    ids, w = oracle.topk_softmax(logits[1:2], 3, True)
    assert ids[0, 0] == 6 and w[0, 0] == 1.0 and np.all(w[0, 1:] == 0)
    assert ids[0, 1:].tolist() == [0, 1]            # the -inf ties by id
    ids, w = oracle.topk_softmax(logits[2:], 8, False)
    assert ids.tolist() == [[7, 6, 5, 4, 3, 2, 1, 0]]
    np.testing.assert_allclose(w.sum(), 1.0, rtol=1e-6)   # K = E: all of the softmax


def test_rejects_bad_sizes():
    with pytest.raises(ValueError):
        oracle.topk_softmax(np.zeros((2, 4), np.float32), 5, True)
