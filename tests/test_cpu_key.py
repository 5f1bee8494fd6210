"""The CPU dispatch key of the drop-in ops (the reference's only key,
Int8-gemm/nanovllm_ops.cpp:410-412), called the way the reference's own
tests call it (Int8-gemm/test/fused_moe_cpu.py:118-160): a MoEInfer handle
loaded from host tensors, then torch.ops.nanovllm.moe_forward on CPU
tensors.

* Q8_0 / Q4_0 run the host engine (the reference CPU algorithm): bit-equal
  to the oracle's fused forward, both loaders (wire repack, online quant).
* W4A16 runs every expert on the host executor: within 1e-5 of the oracle's
  fp32 result before the final cast (different fp32 summation grouping).
* moe_forward_out, moe_topk_softmax and moe_forward_logits on CPU tensors.

Where a HIP device is present the host copy is kept only with
MIMOE_HOST_WEIGHTS=1, which these tests set before creating handles."""
import os

import numpy as np
import pytest
import torch

import oracle
import nanovllm_moe
from helpers import bits, max_rel_err, topk_routing, w4a16_random
from test_oracle_forward import _q_weights


@pytest.fixture(autouse=True)
def _host_weights(monkeypatch):
    monkeypatch.setenv("MIMOE_HOST_WEIGHTS", "1")
    monkeypatch.delenv("NANOVLLM_TP_SIZE", raising=False)
    monkeypatch.delenv("NANOVLLM_TP_THREADS_PER_NODE", raising=False)
    nanovllm_moe.load()


def _q_oracle(qt, x, ids, tw, ws, E, I):
    acode = 1 if x.dtype == torch.bfloat16 else 0
    scode = 1 if ws[1].dtype == torch.bfloat16 else 0
    y, _ = oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids.numpy(),
                                np.asarray(ws[0]), bits(ws[1]), np.asarray(ws[2]), bits(ws[3]), E, I)
    return y


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T,K", [(1, 8), (6, 8), (37, 10), (64, 1)])
def test_moe_forward_cpu_matches_oracle(qt, T, K):
    E, H, I = 16, 256, 128
    ws = _q_weights(qt, E, H, I, 70 + qt, torch.float16 if T % 2 else torch.bfloat16)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, qt)
    h.store_quantized_repack(*[torch.from_numpy(np.ascontiguousarray(t)) if isinstance(t, np.ndarray) else t
                               for t in ws])
    ids, tw = topk_routing(T, E, K, seed=T + K)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
    assert y.dtype == x.dtype and y.shape == x.shape and y.device.type == "cpu"
    assert np.array_equal(bits(y), _q_oracle(qt, x, ids, tw, ws, E, I))
    assert h.get_last_run_time_ms() > 0
    out = torch.empty_like(x)
    torch.ops.nanovllm.moe_forward_out(x, ids, tw, h, out)
    assert torch.equal(out, y)


def test_quantize_and_store_expert_cpu():
    """The reference test's loader (Int8-gemm/test/fused_moe_cpu.py:118-132):
    fp32 weights quantized per expert and projection, then a CPU forward."""
    E, H, I, T, K = 8, 256, 128, 4, 8
    g = torch.Generator().manual_seed(3)
    w13 = torch.randn(E, 2 * I, H, generator=g) * 0.02
    w2 = torch.randn(E, H, I, generator=g) * 0.02
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 0)
    for e in range(E):
        h.quantize_and_store_expert(e, "gate_proj", w13[e, :I].contiguous())
        h.quantize_and_store_expert(e, "up_proj", w13[e, I:].contiguous())
        h.quantize_and_store_expert(e, "down_proj", w2[e].contiguous())
    ids, tw = topk_routing(T, E, K, seed=5)
    x = torch.randn(T, H, generator=g).to(torch.float16)
    y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
    q13, d13 = oracle.quantize_weight_q8_0(w13.reshape(-1, H).numpy())
    q2, d2 = oracle.quantize_weight_q8_0(w2.reshape(-1, I).numpy())
    ws = (q13.reshape(E, 2 * I, H), torch.from_numpy(d13.view(np.float16)).reshape(E, 2 * I, H // 32),
          q2.reshape(E, H, I), torch.from_numpy(d2.view(np.float16)).reshape(E, H, I // 32))
    assert np.array_equal(bits(y), _q_oracle(0, x, ids, tw, ws, E, I))


def test_w4a16_cpu_key():
    E, H, I, T, K = 8, 512, 256, 5, 4
    w = w4a16_random(E, H, I, seed=8)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)
    h.store_awq_repack(*w, 128)
    ids, tw = topk_routing(T, E, K, seed=2)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
    _, yf = oracle.moe_forward_w4a16(1, 1, bits(x), tw.numpy(), ids.numpy(), w[0].numpy(), w[1].numpy(),
                                     bits(w[2]), w[3].numpy(), w[4].numpy(), bits(w[5]), E, I)
    assert max_rel_err(y, torch.from_numpy(yf)) <= 1e-2
    assert max_rel_err(y.float(), torch.from_numpy(yf).to(torch.bfloat16).float()) <= 1e-2


def test_topk_softmax_and_forward_logits_cpu():
    E, H, I, T, K = 16, 256, 128, 9, 8
    logits = torch.randn(T, E, generator=torch.Generator().manual_seed(4))
    logits[0, 3] = logits[0, 5] = logits[0].max() + 1.0      # a tie: the lower id first
    ids, w = torch.ops.nanovllm.moe_topk_softmax(logits, K, True)
    rid, rw = oracle.topk_softmax(logits.numpy(), K, renormalize=True)
    assert np.array_equal(ids.numpy(), rid)
    assert np.array_equal(w.numpy().view(np.uint32), rw.view(np.uint32))   # the device kernel's bits
    assert ids[0, 0] == 3 and ids[0, 1] == 5
    ids_all, w_all = torch.ops.nanovllm.moe_topk_softmax(logits, K, False)
    rid, rw = oracle.topk_softmax(logits.numpy(), K, renormalize=False)
    assert np.array_equal(ids_all.numpy(), rid)
    assert np.array_equal(w_all.numpy().view(np.uint32), rw.view(np.uint32))
    ws = _q_weights(1, E, H, I, 90, torch.float16)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 1)
    h.store_quantized_repack(*[torch.from_numpy(np.ascontiguousarray(t)) if isinstance(t, np.ndarray) else t
                               for t in ws])
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward_logits(x, logits, K, True, h)
    assert torch.equal(y, torch.ops.nanovllm.moe_forward(x, ids, w, h))


def test_cpu_key_argument_errors():
    E, H, I = 8, 256, 128
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 0)
    x = torch.zeros(2, H, dtype=torch.bfloat16)
    ids = torch.zeros(2, 8, dtype=torch.int32)
    w = torch.zeros(2, 8)
    with pytest.raises(RuntimeError, match="not stored|no host weights"):
        torch.ops.nanovllm.moe_forward(x, ids, w, h)
    with pytest.raises(RuntimeError, match="hidden size"):
        torch.ops.nanovllm.moe_forward(torch.zeros(2, H + 32, dtype=torch.bfloat16), ids, w, h)
    with pytest.raises(RuntimeError, match="int32"):
        torch.ops.nanovllm.moe_forward(x, ids.long(), w, h)


def test_reference_device_op_names_on_cpu():
    """The reference's device-op names (Int8-gemm/nanovllm_ops.cpp:393-407):
    moe_forward_npu_stream is moe_forward; moe_forward_npu_graph_out writes
    into out for a MoEGraphContext(moe, num_tokens, top_k, dtype) and rejects
    calls past the context's shape; NpuCallbackManager constructs."""
    E, H, I, T, K = 8, 256, 128, 5, 8
    ws = _q_weights(1, E, H, I, 95, torch.float16)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 1)
    h.store_quantized_repack(*[torch.from_numpy(np.ascontiguousarray(t)) if isinstance(t, np.ndarray) else t
                               for t in ws])
    torch.classes.nanovllm.NpuCallbackManager(0, 0)
    ids, tw = topk_routing(T, E, K, seed=96)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(97)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
    assert torch.equal(torch.ops.nanovllm.moe_forward_npu_stream(x, ids, tw, h), y)
    ctx = torch.classes.nanovllm.MoEGraphContext(h, 8, K, 1)
    out = torch.empty_like(x)
    torch.ops.nanovllm.moe_forward_npu_graph_out(x, ids, tw, h, ctx, out)
    assert torch.equal(out, y)
    with pytest.raises(RuntimeError, match="more tokens"):
        big = torch.zeros(9, H, dtype=torch.bfloat16)
        torch.ops.nanovllm.moe_forward_npu_graph_out(big, torch.zeros(9, K, dtype=torch.int32),
                                                     torch.zeros(9, K), h, ctx, torch.empty_like(big))
    with pytest.raises(RuntimeError, match="top_k"):
        torch.ops.nanovllm.moe_forward_npu_graph_out(x, ids[:, :4].contiguous(), tw[:, :4].contiguous(), h, ctx, out)
    with pytest.raises(RuntimeError, match="dtype"):
        torch.ops.nanovllm.moe_forward_npu_graph_out(x.half(), ids, tw, h, ctx, out.half())
    with pytest.raises(RuntimeError, match="dtype must be"):
        torch.classes.nanovllm.MoEGraphContext(h, 8, K, 2)


def test_reference_env_contract(monkeypatch):
    """NANOVLLM_TP_SIZE / NANOVLLM_TP_THREADS_PER_NODE keep the reference's
    meaning (Int8-gemm/moe_infer.cpp:25-36, Int8-gemm/numa_threadpool.h:498-504,
    README.md:179): with NANOVLLM_TP_SIZE=2 on a one-node host the CPU key runs
    two tp shards, bit-equal to the oracle at tp=2 (whose shard-order sum
    differs from tp=1 here); tp_size 0 is refused as in the reference."""
    E, H, I, T, K, qt = 16, 1024, 512, 16, 8, 0
    ws = _q_weights(qt, E, H, I, 4, torch.float16)
    ids, tw = topk_routing(T, E, K, seed=5)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(6)).to(torch.float16)
    acode, scode = 0, 0
    refs = {tp: oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids.numpy(), np.asarray(ws[0]),
                                     bits(ws[1]), np.asarray(ws[2]), bits(ws[3]), E, I, tp=tp)[0] for tp in (1, 2)}
    assert not np.array_equal(refs[1], refs[2])
    load = lambda h: h.store_quantized_repack(*[torch.from_numpy(np.ascontiguousarray(t))
                                                if isinstance(t, np.ndarray) else t for t in ws])
    monkeypatch.setenv("NANOVLLM_TP_SIZE", "2")
    monkeypatch.setenv("NANOVLLM_TP_THREADS_PER_NODE", "2")
    h = torch.classes.nanovllm.MoEInfer(E, H, I, qt)
    load(h)
    y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
    assert np.array_equal(bits(y), refs[2])
    monkeypatch.setenv("NANOVLLM_TP_SIZE", "0")
    with pytest.raises(RuntimeError, match="tp_size must be >= 1"):   # when the host engine is made
        h0 = torch.classes.nanovllm.MoEInfer(E, H, I, qt)
        load(h0)
        torch.ops.nanovllm.moe_forward(x, ids, tw, h0)
