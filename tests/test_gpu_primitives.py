"""GPU parity of the integer primitives through the C ABI, bit-exact against
the oracle: routing (preprocess_moe_routing, Int8-gemm/moe_common.cpp:
146-216) and Stage A Q8_0 activation quantization (Int8-gemm/q8_gemm.cpp:
360-377, gemm_kernels.cpp:25-58)."""
import ctypes

import numpy as np
import pytest
import torch

import nanovllm_moe
import oracle
from helpers import bits

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


@pytest.mark.parametrize("T,K,E,seed", [(1, 8, 128, 0), (8, 8, 128, 1), (128, 8, 128, 2),
                                        (4096, 8, 128, 3), (512, 8, 256, 4), (300, 10, 64, 5),
                                        (77, 1, 16, 6), (0, 8, 128, 7),
                                        # multi-workgroup routing (> 4096 pairs): ragged last
                                        # chunk, and the largest expert count
                                        (700, 8, 128, 8), (1100, 10, 512, 9)])
def test_route_bit_exact(cuda, T, K, E, seed):
    rng = np.random.default_rng(seed)
    ids = rng.integers(-1, E + 1, size=(T, K)).astype(np.int32)
    if T > 2:
        ids[1, :] = 3                       # duplicates inside a token
    L = nanovllm_moe.capi()
    d_ids = torch.from_numpy(ids).to(cuda)
    counts = torch.zeros(E, dtype=torch.int32, device=cuda)
    starts = torch.zeros(E + 1, dtype=torch.int32, device=cuda)
    n = max(T * K, 1)
    tmap = torch.full((n,), -7, dtype=torch.int32, device=cuda)
    scat = torch.full((n,), -7, dtype=torch.int32, device=cuda)
    rc = L.mi_moe_route(_ptr(d_ids), T, K, E, _ptr(counts), _ptr(starts), _ptr(tmap), _ptr(scat),
                        nanovllm_moe.stream_ptr())
    nanovllm_moe.check(rc, "mi_moe_route")
    torch.cuda.synchronize()
    c_ref, s_ref, tm_ref, sc_ref = oracle.route(ids, E)
    assert np.array_equal(counts.cpu().numpy(), c_ref)
    assert np.array_equal(starts.cpu().numpy(), s_ref)
    nv = int(s_ref[E])
    assert np.array_equal(tmap.cpu().numpy()[:nv], tm_ref[:, 0])
    if T:
        assert np.array_equal(scat.cpu().numpy()[:T * K].reshape(T, K), sc_ref)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T,H", [(1, 2048), (8, 2048), (513, 3072), (4096, 2048)])
def test_quant_act_bit_exact(cuda, dt, T, H):
    g = torch.Generator().manual_seed(T + H)
    x = (torch.randn(T, H, generator=g) * 3).to(dt)
    if T >= 8:
        x[1] = 0                                        # all-zero blocks
        x[2, :32] = torch.tensor([127.0] + [0.5, 1.5, 2.5, 3.5, -2.5] + [0.0] * 26).to(dt)  # ties
        x[3] = x[3] * 1000
    code = nanovllm_moe.dtype_code(dt)
    xd = x.to(cuda)
    qs = torch.empty(T, H, dtype=torch.int8, device=cuda)
    d = torch.empty(T, H // 32, dtype=torch.float32, device=cuda)
    L = nanovllm_moe.capi()
    nanovllm_moe.check(L.mi_moe_quantize_act_q8_0(_ptr(xd), code, T, H, _ptr(qs), _ptr(d),
                                                  nanovllm_moe.stream_ptr()), "quantize_act")
    torch.cuda.synchronize()
    q_ref, d_ref = oracle.quantize_act_q8_0(bits(x), code)
    assert np.array_equal(qs.cpu().numpy(), q_ref)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), d_ref.view(np.uint32))
