"""GPU parity of the hybrid offload executor (mi_moe_hybrid_forward through
nanovllm_moe.HybridMoE): hot experts run by the device kernels, cold experts
by host threads in a stream host callback, the fp32 partial added on the
device.  The oracle's fused forward over all experts is the reference
(Int8-gemm/q8_gemm.cpp:276-646; the W4A16 restatement).  Tolerance: the
north-star max|y - y_ref| / max|y_ref| <= 1e-2 on the 16-bit output (the
device partial is rounded to the activation dtype before the add)."""
import numpy as np
import pytest
import torch

import nanovllm_moe as nm
import oracle
from nanovllm_moe import HybridMoE
from helpers import bits, max_rel_err, topk_routing, w4a16_random
from test_oracle_forward import _q_weights

pytestmark = pytest.mark.gpu
TOL = 1e-2
W4 = dict(E=16, H=512, I=256)
Q = dict(E=16, H=256, I=128)
COLD = [1, 2, 5, 11, 15]


def _x(T, H, seed):
    return (torch.randn(T, H, generator=torch.Generator().manual_seed(seed)) * 0.7).to(torch.bfloat16)


def _oracle_w4(x, ids, tw, ws, E, I):
    _, yf = oracle.moe_forward_w4a16(1, 1 if ws[2].dtype == torch.bfloat16 else 0, bits(x), tw.numpy(),
                                     ids.numpy(), ws[0].numpy(), ws[1].numpy(), bits(ws[2]), ws[3].numpy(),
                                     ws[4].numpy(), bits(ws[5]), E, I, nthreads=8)
    return torch.from_numpy(yf)


def _oracle_q(qt, x, ids, tw, ws, E, I):
    _, yf = oracle.moe_forward_q(qt, 1, 1 if ws[1].dtype == torch.bfloat16 else 0, bits(x), tw.numpy(),
                                 ids.numpy(), ws[0], bits(ws[1]), ws[2], bits(ws[3]), E, I)
    return torch.from_numpy(yf)


def _fwd(hm, x, ids, tw, cuda):
    y = hm.forward(x.to(cuda), ids.to(cuda), tw.to(cuda))
    torch.cuda.synchronize()
    return y.cpu()


@pytest.fixture(scope="module")
def w4w():
    return w4a16_random(W4["E"], W4["H"], W4["I"], seed=200)


@pytest.fixture(scope="module")
def w4h(cuda, w4w):
    hm = HybridMoE(W4["E"], W4["H"], W4["I"], nm.W4A16, host_experts=COLD, num_threads=4)
    hm.store_awq(*w4w)
    return hm


@pytest.mark.parametrize("T,K", [(1, 8), (4, 8), (8, 8), (40, 4), (130, 8)])
def test_w4a16_hybrid_parity(cuda, w4w, w4h, T, K):
    E, H, I = W4["E"], W4["H"], W4["I"]
    ids, tw = topk_routing(T, E, K, seed=300 + T + K)
    x = _x(T, H, T)
    y = _fwd(w4h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle_w4(x, ids, tw, w4w, E, I)) <= TOL
    st = w4h.stats()
    assert st["device_experts"] == E - len(COLD) and st["host_experts"] == len(COLD)
    assert st["last_host_pairs"] == int(np.isin(ids.numpy(), COLD).sum())


def test_w4a16_hybrid_device_sources_and_all_device_agree(cuda, w4w):
    """Weights stored from HIP tensors; the hybrid and an all-device handle agree."""
    E, H, I = W4["E"], W4["H"], W4["I"]
    hm = HybridMoE(E, H, I, nm.W4A16, host_experts=[0, 7, 8], num_threads=2)
    hm.store_awq(*[t.to(cuda) for t in w4w])
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)
    h.store_awq_repack(*w4w, 128)
    ids, tw = topk_routing(8, E, 8, seed=310)
    x = _x(8, H, 311)
    y = _fwd(hm, x, ids, tw, cuda)
    y_dev = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h).cpu()
    assert max_rel_err(y, y_dev.float()) <= TOL
    assert max_rel_err(y, _oracle_w4(x, ids, tw, w4w, E, I)) <= TOL


def test_w4a16_all_host_and_all_device_handles(cuda, w4w):
    E, H, I = W4["E"], W4["H"], W4["I"]
    ids, tw = topk_routing(5, E, 8, seed=320)
    x = _x(5, H, 321)
    ref = _oracle_w4(x, ids, tw, w4w, E, I)
    cold = HybridMoE(E, H, I, nm.W4A16, host_experts=range(E), num_threads=4)
    cold.store_awq(*w4w)
    assert max_rel_err(_fwd(cold, x, ids, tw, cuda), ref) <= TOL
    hot = HybridMoE(E, H, I, nm.W4A16, host_experts=[], num_threads=1)
    hot.store_awq(*w4w)
    y_hot = _fwd(hot, x, ids, tw, cuda)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)
    h.store_awq_repack(*w4w, 128)
    y_dev = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h).cpu()
    assert torch.equal(y_hot, y_dev)   # no cold expert: the device handle's forward, unchanged


def test_w4a16_back_to_back_calls(cuda, w4w, w4h):
    """Calls queued without a synchronization in between (the staging buffers
    are reused in stream order), invalid ids included."""
    E, H, I = W4["E"], W4["H"], W4["I"]
    cases = []
    for i, T in enumerate((16, 3, 9, 1)):
        ids, tw = topk_routing(T, E, 8, seed=330 + i)
        ids = ids.clone()
        ids[0, 0] = -1
        cases.append((_x(T, H, 340 + i), ids, tw))
    outs = [w4h.forward(x.to(cuda), ids.to(cuda), tw.to(cuda)) for x, ids, tw in cases]
    torch.cuda.synchronize()
    for (x, ids, tw), y in zip(cases, outs):
        assert max_rel_err(y.cpu(), _oracle_w4(x, ids, tw, w4w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T", [1, 8, 40])
def test_q_hybrid_parity(cuda, qt, T):
    E, H, I = Q["E"], Q["H"], Q["I"]
    ws = _q_weights(qt, E, H, I, 400 + qt, torch.float16)
    hm = HybridMoE(E, H, I, qt, host_experts=COLD, num_threads=4)
    hm.store_quantized(torch.from_numpy(np.ascontiguousarray(ws[0])), ws[1],
                       torch.from_numpy(np.ascontiguousarray(ws[2])), ws[3])
    ids, tw = topk_routing(T, E, 8, seed=410 + T)
    x = _x(T, H, 411 + T)
    y = _fwd(hm, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle_q(qt, x, ids, tw, ws, E, I)) <= TOL


@pytest.mark.parametrize("kind", ["w4a16", "q8_0", "q4_0"])
def test_hybrid_graph_replay_matches_eager(cuda, w4w, kind):
    """Hybrid calls captured into a HIP graph (after one eager call of the
    size, which sizes the staging buffers and the device workspace): the
    device kernels, the staging kernel, the host callback node and the add
    kernel replay bit-identical to the eager calls, with eager calls on the
    same handle between the replays."""
    if kind == "w4a16":
        E, H, I = W4["E"], W4["H"], W4["I"]
        hm = HybridMoE(E, H, I, nm.W4A16, host_experts=COLD, num_threads=4)
        hm.store_awq(*w4w)
    else:
        qt = 0 if kind == "q8_0" else 1
        E, H, I = Q["E"], Q["H"], Q["I"]
        ws = _q_weights(qt, E, H, I, 420 + qt, torch.float16)
        hm = HybridMoE(E, H, I, qt, host_experts=COLD, num_threads=4)
        hm.store_quantized(torch.from_numpy(np.ascontiguousarray(ws[0])), ws[1],
                           torch.from_numpy(np.ascontiguousarray(ws[2])), ws[3])
    cases = []
    for s, T in enumerate((6, 3)):
        ids, tw = topk_routing(T, E, 8, seed=430 + s)
        cases.append((_x(T, H, 440 + s).to(cuda), ids.to(cuda), tw.to(cuda)))
    outs = [torch.empty(x.shape, dtype=torch.bfloat16, device=cuda) for x, _, _ in cases]
    for (x, ids, tw), o in zip(cases, outs):
        hm.forward(x, ids, tw, out=o)
    torch.cuda.synchronize()
    eager = [o.clone() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for (x, ids, tw), o in zip(cases, outs):
            hm.forward(x, ids, tw, out=o)
    for rep in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e), f"replay {rep}"
        x, ids, tw = cases[rep % 2]
        y = hm.forward(x, ids, tw)
        torch.cuda.synchronize()
        assert torch.equal(y, eager[rep % 2])
    del g


def test_hybrid_graph_survives_staging_growth(cuda, w4w):
    """A captured hybrid call keeps its staging buffers and its callback's view
    of them: a later, larger eager call grows the staging (and the device
    workspace) without freeing what the graph holds, and the graph still
    replays the eager result bit for bit."""
    E, H, I = W4["E"], W4["H"], W4["I"]
    hm = HybridMoE(E, H, I, nm.W4A16, host_experts=COLD, num_threads=4)
    hm.store_awq(*w4w)
    T, K = 4, 8
    ids, tw = topk_routing(T, E, K, seed=450)
    x, ids, tw = _x(T, H, 451).to(cuda), ids.to(cuda), tw.to(cuda)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=cuda)
    hm.forward(x, ids, tw, out=out)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        hm.forward(x, ids, tw, out=out)
    T2 = 64                                        # staging capacity 16 tokens / 128 pairs: grows
    ids2, tw2 = topk_routing(T2, E, K, seed=452)
    y2 = hm.forward(_x(T2, H, 453).to(cuda), ids2.to(cuda), tw2.to(cuda))
    torch.cuda.synchronize()
    assert torch.isfinite(y2.float()).all()
    for rep in range(2):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
    del g
