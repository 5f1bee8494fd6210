"""mi_moe_forward_noalloc (the allocation-free variant of mi_moe_forward:
workspace in a static per-GPU device array) against mi_moe_forward, through
the C ABI: the same kernels run on the same inputs, so the outputs must be
bit-identical.  Two calls in a row on each path, the second with a smaller
input (the array keeps the first call's contents), decode and sorted paths of
both formats, and a call too large for the array refused with a status."""
import ctypes

import numpy as np
import pytest
import torch

import nanovllm_moe
from helpers import topk_routing, w4a16_random
import nanovllm_moe.formats as fmt

pytestmark = pytest.mark.gpu


def _handle(L, E, H, I, qt, cuda, seed):
    hp = ctypes.c_void_p()
    nanovllm_moe.check(L.mi_moe_create(E, H, I, qt, ctypes.byref(hp)), "create")
    g = torch.Generator().manual_seed(seed)
    if qt == 2:
        ws = [t.to(cuda) for t in w4a16_random(E, H, I, seed=seed)]
        nanovllm_moe.check(L.mi_moe_store_awq(hp, *[t.data_ptr() for t in ws], 128, nanovllm_moe.BF16, 1,
                                              nanovllm_moe.stream_ptr()), "store_awq")
    else:
        q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g, scale_dtype=torch.float16)
        q2, d2 = fmt.q4_0_random((E, H), I, generator=g, scale_dtype=torch.float16)
        ws = [t.contiguous().to(cuda) for t in (q13, d13, q2, d2)]
        nanovllm_moe.check(L.mi_moe_store_quantized(hp, *[t.data_ptr() for t in ws], nanovllm_moe.F16, 1,
                                                    nanovllm_moe.stream_ptr()), "store_quantized")
    torch.cuda.synchronize()
    return hp


def _call(L, fn, hp, x, ids, tw):
    y = torch.full_like(x, float("nan"))
    rc = fn(hp, x.data_ptr(), y.data_ptr(), tw.data_ptr(), ids.data_ptr(), x.shape[0], ids.shape[1],
            nanovllm_moe.dtype_code(x.dtype), nanovllm_moe.stream_ptr())
    nanovllm_moe.check(rc, fn.__name__)
    return y


# (T, K) of the two calls: the second smaller.  W4A16 (E=8, H=512, I=256):
# 40x8 = 320 pairs takes the sorted path, 3x4 the decode path; Q4_0: 24x8 the
# int8 grouped GEMMs, 16x8 and 2x8 the lane-per-row kernels.
@pytest.mark.parametrize("qt,calls", [(2, [(40, 8), (3, 4)]), (2, [(8, 8), (1, 8)]),
                                      (1, [(24, 8), (2, 8)]), (1, [(16, 8), (1, 4)])])
def test_noalloc_matches_forward(cuda, qt, calls):
    L = nanovllm_moe.capi()
    E, H, I = 8, 512, 256
    hp = _handle(L, E, H, I, qt, cuda, seed=70 + qt)
    try:
        for i, (T, K) in enumerate(calls):
            print(f"[no_alloc] qt={qt} call {i}: T={T} K={K}", flush=True)
            ids, tw = topk_routing(T, E, K, seed=100 * i + T)
            ids, tw = ids.to(cuda), tw.to(cuda)
            x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).to(cuda)
            ref = _call(L, L.mi_moe_forward, hp, x, ids, tw)
            got = _call(L, L.mi_moe_forward_noalloc, hp, x, ids, tw)
            torch.cuda.synchronize()
            assert torch.isfinite(ref.float()).all()
            assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (qt, T, K)
    finally:
        L.mi_moe_destroy(hp)


def test_noalloc_rejects_oversize_call(cuda):
    """A sorted-path call whose per-pair fp32 outputs alone exceed the array:
    refused before any launch, with the sizes in the message."""
    L = nanovllm_moe.capi()
    E, H, I = 8, 512, 256
    hp = _handle(L, E, H, I, 2, cuda, seed=3)
    try:
        T, K = 2048, 8                     # 16384 pairs x 512 x 4 B = 32 MiB of outputs alone
        ids, tw = topk_routing(T, E, K, seed=1)
        x = torch.zeros(T, H, dtype=torch.bfloat16, device=cuda)
        y = torch.empty_like(x)
        rc = L.mi_moe_forward_noalloc(hp, x.data_ptr(), y.data_ptr(), tw.to(cuda).data_ptr(),
                                      ids.to(cuda).data_ptr(), T, K, nanovllm_moe.BF16, nanovllm_moe.stream_ptr())
        assert rc == 1
        assert b"mi_moe_forward_noalloc holds at most" in L.mi_moe_last_error()
    finally:
        L.mi_moe_destroy(hp)


def test_noalloc_keeps_phase_times(cuda):
    """A no-alloc call records no timing and leaves the phase times of the last
    timed mi_moe_forward as they were (2 phases for a sorted-path call)."""
    L = nanovllm_moe.capi()
    E, H, I = 8, 512, 256
    hp = _handle(L, E, H, I, 2, cuda, seed=5)
    try:
        nanovllm_moe.check(L.mi_moe_set_timing(hp, 1), "set_timing")
        T, K = 40, 8                       # 320 pairs: the sorted path, two launch phases
        ids, tw = topk_routing(T, E, K, seed=4)
        ids, tw = ids.to(cuda), tw.to(cuda)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16).to(cuda)
        _call(L, L.mi_moe_forward, hp, x, ids, tw)
        ms = (ctypes.c_double * 2)()
        assert L.mi_moe_get_last_phase_times_ms(hp, ms, 2) == 2
        _call(L, L.mi_moe_forward_noalloc, hp, x[:3], ids[:3].contiguous(), tw[:3].contiguous())
        torch.cuda.synchronize()
        assert L.mi_moe_get_last_phase_times_ms(hp, ms, 2) == 2
    finally:
        L.mi_moe_destroy(hp)
