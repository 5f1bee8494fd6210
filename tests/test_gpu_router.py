"""GPU router top-k + softmax (mi_moe_topk_softmax; the reference's
make_topk_from_logits_cpu, Int8-gemm/test/fused_moe_cpu.py:20-37) against the
oracle: ids and weights bit-exact (same exp restatement, sums in the same
order, IEEE division), fp32 / bf16 / fp16 logits, both softmax modes, ties;
and moe_forward_logits equal to topk + moe_forward."""
import ctypes

import numpy as np
import pytest
import torch

import nanovllm_moe
import oracle
from helpers import w4a16_random

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _gpu_topk(logits, K, renorm, cuda):
    L = nanovllm_moe.capi()
    g = logits.to(cuda).contiguous()
    T, E = g.shape
    ids = torch.full((T, K), -7, dtype=torch.int32, device=cuda)
    w = torch.full((T, K), -7.0, dtype=torch.float32, device=cuda)
    code = {torch.float32: nanovllm_moe.F32, torch.bfloat16: nanovllm_moe.BF16, torch.float16: nanovllm_moe.F16}
    rc = L.mi_moe_topk_softmax(_ptr(g), code[g.dtype], T, E, K, 1 if renorm else 0, _ptr(ids), _ptr(w),
                               nanovllm_moe.stream_ptr())
    nanovllm_moe.check(rc, "mi_moe_topk_softmax")
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy()


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("T,E,K", [(1, 128, 8), (8, 128, 8), (33, 256, 10), (4096, 128, 8),
                                   (5, 512, 64), (3, 16, 16), (7, 100, 1)])
def test_topk_softmax_bit_exact(cuda, dt, renorm, T, E, K):
    g = torch.Generator().manual_seed(T * 1000 + E + K)
    logits = (torch.randn(T, E, generator=g) * 3).to(dt)
    ids, w = _gpu_topk(logits, K, renorm, cuda)
    rid, rw = oracle.topk_softmax(logits.float().numpy(), K, renorm)
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))


def test_topk_softmax_ties_and_edges(cuda):
    logits = torch.zeros(4, 64)
    logits[0, [1, 2, 40, 63]] = 5.0                 # four-way tie across lanes
    logits[1] = -float("inf")
    logits[1, 50] = 0.0                             # one finite logit, rest -inf
    logits[2] = torch.arange(64, dtype=torch.float32) % 3   # many ties
    logits[3] = 0.0                                 # all equal
    for renorm in (True, False):
        ids, w = _gpu_topk(logits, 8, renorm, cuda)
        rid, rw = oracle.topk_softmax(logits.numpy(), 8, renorm)
        assert np.array_equal(ids, rid)
        assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    assert ids[0, :4].tolist() == [1, 2, 40, 63] and ids[3].tolist() == list(range(8))


@pytest.mark.parametrize("quant", [1, 2])
@pytest.mark.parametrize("T", [3, 40])
def test_forward_logits_equals_two_step(cuda, quant, T):
    E, H, I, K = 16, 512, 256, 8
    g = torch.Generator().manual_seed(T + quant)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, quant)
    if quant == 2:
        h.store_awq_repack(*[t.to(cuda) for t in w4a16_random(E, H, I, seed=T)], 128)
    else:
        import nanovllm_moe.formats as fmt
        q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g)
        q2, d2 = fmt.q4_0_random((E, H), I, generator=g)
        h.store_quantized_repack(q13.to(cuda), d13.to(cuda), q2.to(cuda), d2.to(cuda))
    x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda)
    logits = torch.randn(T, E, generator=g).to(cuda)
    y1 = torch.ops.nanovllm.moe_forward_logits(x, logits, K, True, h)
    ids, w = torch.ops.nanovllm.moe_topk_softmax(logits, K, True)
    y2 = torch.ops.nanovllm.moe_forward(x, ids, w, h)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    rid, rw = oracle.topk_softmax(logits.cpu().numpy(), K, True)
    assert np.array_equal(ids.cpu().numpy(), rid)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("E,T,K", [(16, 3, 8), (128, 1, 8), (128, 8, 8), (128, 6, 10), (512, 2, 16), (64, 64, 1)])
def test_forward_logits_decode_router_pass(cuda, dt, renorm, E, T, K):
    """mi_moe_forward_logits on W4A16 decode sizes, every logits dtype and
    softmax mode: the ids and weights it returns are bit-exact against the
    oracle, and y equals mi_moe_forward on them bit for bit."""
    H, I = 512, 256
    L = nanovllm_moe.capi()
    g = torch.Generator().manual_seed(E * 100 + T * 10 + K)
    hp = ctypes.c_void_p()
    nanovllm_moe.check(L.mi_moe_create(E, H, I, 2, ctypes.byref(hp)), "create")
    try:
        ws = [t.to(cuda) for t in w4a16_random(E, H, I, seed=E + T)]
        nanovllm_moe.check(L.mi_moe_store_awq(hp, *[t.data_ptr() for t in ws], 128, nanovllm_moe.BF16, 1,
                                              nanovllm_moe.stream_ptr()), "store_awq")
        x = torch.randn(T, H, generator=g).to(torch.bfloat16).to(cuda)
        logits = (torch.randn(T, E, generator=g) * 2).to(dt).to(cuda)
        ids = torch.full((T, K), -7, dtype=torch.int32, device=cuda)
        w = torch.full((T, K), -7.0, dtype=torch.float32, device=cuda)
        y1 = torch.full_like(x, float("nan"))
        code = {torch.float32: nanovllm_moe.F32, torch.bfloat16: nanovllm_moe.BF16,
                torch.float16: nanovllm_moe.F16}
        rc = L.mi_moe_forward_logits(hp, _ptr(x), _ptr(y1), _ptr(logits), code[dt], T, K, 1 if renorm else 0,
                                     nanovllm_moe.BF16, _ptr(ids), _ptr(w), nanovllm_moe.stream_ptr())
        nanovllm_moe.check(rc, "mi_moe_forward_logits")
        torch.cuda.synchronize()
        rid, rw = oracle.topk_softmax(logits.float().cpu().numpy(), K, renorm)
        assert np.array_equal(ids.cpu().numpy(), rid)
        assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
        y2 = torch.full_like(x, float("nan"))
        nanovllm_moe.check(L.mi_moe_forward(hp, _ptr(x), _ptr(y2), _ptr(w), _ptr(ids), T, K, nanovllm_moe.BF16,
                                            nanovllm_moe.stream_ptr()), "mi_moe_forward")
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
    finally:
        L.mi_moe_destroy(hp)
