"""Top-10 routing on the decode path (the reference's Q4_0 benchmark shape,
Int8-gemm/test/benchmark_fused_moe_int4.py:12-15: H=2048, I=512, E=128,
top-10, token counts 1..8).

Q8_0 / Q4_0 calls of up to 96 / 160 routed pairs run the lane-per-row
kernels with the token-major down kernel (one wave per routed expert of a
token, up to 16) -- every T of the benchmark; above, the int8 grouped GEMMs.
W4A16 calls of up to 64 pairs (T <= 6) run the two decode launches, T = 7
the sorted path.  Parity is against the oracle
on the same inputs, max-rel-err <= 1e-2 (the fp32 sums differ only in their
wave-split order), with both the reference benchmark's round-robin routing
(ids[t,k] = (t*K + k) % E, weights 1/K;
Int8-gemm/test/benchmark_fused_moe_cpu.py:171-178) and seeded random top-10
routing with renormalized softmax weights, invalid ids included.  The kernels
a call launches are read from the torch profiler's device trace where it
records one."""
import numpy as np
import pytest
import torch

import oracle
from helpers import bits, max_rel_err, topk_routing, w4a16_random
import nanovllm_moe.formats as fmt

pytestmark = pytest.mark.gpu
TOL = 1e-2
E, H, I, K = 128, 2048, 512, 10


def _round_robin(T, K, E):
    ids = ((torch.arange(T)[:, None] * K + torch.arange(K)[None, :]) % E).to(torch.int32)
    return ids, torch.full((T, K), 1.0 / K, dtype=torch.float32)


def _q_weights(qt, seed):
    g = torch.Generator().manual_seed(seed)
    if qt == 0:
        w13 = torch.randn(E, 2 * I, H, generator=g) * 0.02
        w2 = torch.randn(E, H, I, generator=g) * 0.02
        q13, d13 = oracle.quantize_weight_q8_0(w13.reshape(-1, H).numpy())
        q2, d2 = oracle.quantize_weight_q8_0(w2.reshape(-1, I).numpy())
        return (torch.from_numpy(q13.reshape(E, 2 * I, H)),
                torch.from_numpy(d13.view(np.float16)).reshape(E, 2 * I, H // 32),
                torch.from_numpy(q2.reshape(E, H, I)),
                torch.from_numpy(d2.view(np.float16)).reshape(E, H, I // 32))
    q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g)
    q2, d2 = fmt.q4_0_random((E, H), I, generator=g)
    return q13, d13, q2, d2


@pytest.fixture(scope="module")
def q_layers(cuda):
    out = {}
    for qt in (0, 1):
        w = _q_weights(qt, 500 + qt)
        h = torch.classes.nanovllm.MoEInfer(E, H, I, qt)
        h.store_quantized_repack(*[t.to(cuda) for t in w])
        out[qt] = (w, h)
    return out


def _q_oracle(qt, x, ids, tw, w):
    _, yf = oracle.moe_forward_q(qt, 1, 0, bits(x), tw.numpy(), ids.numpy(), w[0].numpy(), bits(w[1]),
                                 w[2].numpy(), bits(w[3]), E, I)
    return torch.from_numpy(yf)


def _run(h, x, ids, tw, cuda):
    y = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h)
    torch.cuda.synchronize()
    return y.cpu()


def _kernels(fn):
    """Names of the device kernels fn launches, from the torch profiler's
    device trace (None if the trace holds no kernels)."""
    from torch.profiler import ProfilerActivity, profile
    with profile(activities=[ProfilerActivity.CUDA]) as p:
        fn()
        torch.cuda.synchronize()
    names = [e.name for e in p.events() if e.device_type == torch.autograd.DeviceType.CUDA]
    names = [n for n in names if "kernel" in n.lower()]
    return names or None


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T", [1, 2, 3, 4, 5, 6, 7, 8])
def test_q_top10_round_robin(cuda, q_layers, qt, T):
    w, h = q_layers[qt]
    ids, tw = _round_robin(T, K, E)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _q_oracle(qt, x, ids, tw, w)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T", [1, 4, 6, 12, 17])
def test_q_top10_random_routing_invalid_ids(cuda, q_layers, qt, T):
    w, h = q_layers[qt]
    ids, tw = topk_routing(T, E, K, seed=90 + T)
    ids = ids.clone()
    ids[0, 9] = -1                       # dropped pair
    if T >= 4:
        ids[2, :] = E + 3                # a token with no valid id: y = 0
        ids[3, 0] = ids[3, 1]            # a token routed twice to one expert
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T + 7)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _q_oracle(qt, x, ids, tw, w)) <= TOL
    if T >= 4:
        assert torch.all(y[2] == 0)


@pytest.fixture(scope="module")
def w4_layer(cuda):
    Ew, Hw, Iw = 32, 2048, 768
    w = w4a16_random(Ew, Hw, Iw, seed=510)
    h = torch.classes.nanovllm.MoEInfer(Ew, Hw, Iw, 2)
    h.store_awq_repack(*[t.to(cuda) for t in w], 128)
    return w, h, (Ew, Hw, Iw)


@pytest.mark.parametrize("T", [1, 3, 6, 7])
def test_w4a16_top10(cuda, w4_layer, T):
    w, h, (Ew, Hw, Iw) = w4_layer
    ids, tw = topk_routing(T, Ew, K, seed=30 + T)
    ids = ids.clone()
    ids[T - 1, 4] = -1
    x = torch.randn(T, Hw, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    w13_q, w13_z, w13_s, w2_q, w2_z, w2_s = w
    _, yf = oracle.moe_forward_w4a16(1, 1, bits(x), tw.numpy(), ids.numpy(), w13_q.numpy(), w13_z.numpy(),
                                     bits(w13_s), w2_q.numpy(), w2_z.numpy(), bits(w2_s), Ew, Iw, nthreads=8)
    assert max_rel_err(y, torch.from_numpy(yf)) <= TOL


def test_top10_decode_launches(cuda, q_layers, w4_layer):
    """The kernels a top-10 call launches: Q4_0 at 8 and 16 tokens (80, 160
    pairs) and Q8_0 at 8 tokens the lane-per-row kernels with the token-major
    down (combine fused), no routing or grouped-GEMM kernel; Q4_0 at 17 and
    Q8_0 at 10 tokens the grouped GEMMs; W4A16 at 6 tokens the two decode
    launches, at 7 the sorted path."""
    _, hw, (Ew, Hw, _) = w4_layer
    cases = []
    for qt, T, decode in ((1, 8, True), (1, 16, True), (1, 17, False), (0, 8, True), (0, 10, False)):
        ids, tw = _round_robin(T, K, E)
        x = torch.randn(T, H, dtype=torch.bfloat16, device=cuda)
        cases.append((decode, q_layers[qt][1], x, ids.to(cuda), tw.to(cuda)))
    for T in (6, 7):
        idw, tww = topk_routing(T, Ew, K, seed=T)
        xw = torch.randn(T, Hw, dtype=torch.bfloat16, device=cuda)
        cases.append((T == 6, hw, xw, idw.to(cuda), tww.to(cuda)))
    for decode, h, x, ids, tw in cases:
        torch.ops.nanovllm.moe_forward(x, ids, tw, h)   # warm (LDS opt-in, workspace)
        names = _kernels(lambda: torch.ops.nanovllm.moe_forward(x, ids, tw, h))
        if names is None:
            pytest.skip("the profiler recorded no device kernels on this system")
        joined = " ".join(names)
        if decode:
            assert "down_token" in joined, names
            assert "gemm" not in joined and "route" not in joined, names
        else:
            assert "gemm" in joined, names
