"""GPU parity at the BASELINE configurations beyond the headline one, at
their full sizes:

* config 3, Q4_0 prefill, Qwen3 shape (E=128, H=2048, I=768, top-8),
  T = 32 / 128 / 1024 / 4096;
* config 4, MiniMax-M2 W4A16 shape (E=256, H=3072, I=1536, top-8) at bs 64
  (the sorted-routing path; bs 1 and 8 are in test_gpu_w4a16.py);
* config 5, Zipf-skewed routing (p ~ r^-1.2) at T = 512 on the Qwen3 W4A16
  shape, where the hottest experts take hundreds of rows.

The layer is token-independent (routing, activation quantization, the
intermediate and the combine are all per token or per pair), so the oracle
is run on a seeded sample of tokens and compared with the same rows of the
full GPU output (max-rel-err <= 1e-2 over the sample, as elsewhere)."""
import pytest
import torch

import oracle
import nanovllm_moe.formats as fmt
from helpers import bits, max_rel_err, token_sample, topk_routing, w4a16_random, zipf_routing

pytestmark = pytest.mark.gpu
TOL = 1e-2
QWEN = dict(E=128, H=2048, I=768)


@pytest.fixture(scope="module")
def q4_qwen(cuda):
    E, H, I = QWEN["E"], QWEN["H"], QWEN["I"]
    g = torch.Generator().manual_seed(0)
    q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g)
    q2, d2 = fmt.q4_0_random((E, H), I, generator=g)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 1)
    h.store_quantized_repack(q13.to(cuda), d13.to(cuda), q2.to(cuda), d2.to(cuda))
    return (q13, d13, q2, d2), h


@pytest.mark.parametrize("T", [32, 128, 1024, 4096])
def test_config3_q4_0_prefill(cuda, q4_qwen, T):
    (q13, d13, q2, d2), h = q4_qwen
    E, H, I = QWEN["E"], QWEN["H"], QWEN["I"]
    ids, tw = topk_routing(T, E, 8, seed=300 + T)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h)
    torch.cuda.synchronize()
    y = y.cpu()
    s = token_sample(T, 24, seed=T)
    _, ref = oracle.moe_forward_q(1, 1, 0, bits(x[s]), tw[s].numpy(), ids[s].numpy(), q13.numpy(),
                                  bits(d13), q2.numpy(), bits(d2), E, I)
    assert max_rel_err(y[s], torch.from_numpy(ref)) <= TOL


def _w4a16_oracle(x, ids, tw, w, E, I):
    w13_q, w13_z, w13_s, w2_q, w2_z, w2_s = w
    _, yf = oracle.moe_forward_w4a16(1, 1, bits(x), tw.numpy(), ids.numpy(), w13_q.numpy(), w13_z.numpy(),
                                     bits(w13_s), w2_q.numpy(), w2_z.numpy(), bits(w2_s), E, I, nthreads=8)
    return torch.from_numpy(yf)


def test_config4_minimax_bs64(cuda):
    E, H, I = 256, 3072, 1536
    w = w4a16_random(E, H, I, seed=4)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)
    h.store_awq_repack(*[t.to(cuda) for t in w], 128)
    T = 64
    ids, tw = topk_routing(T, E, 8, seed=64)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(64)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h)
    torch.cuda.synchronize()
    s = token_sample(T, 16, seed=64)
    assert max_rel_err(y.cpu()[s], _w4a16_oracle(x[s], ids[s], tw[s], w, E, I)) <= TOL


def test_config5_zipf_skew(cuda):
    E, H, I = QWEN["E"], QWEN["H"], QWEN["I"]
    T, K = 512, 8
    ids, tw = zipf_routing(T, E, K, seed=0)
    counts = torch.bincount(ids.reshape(-1).long(), minlength=E)
    # the skew the configuration is about: the hottest expert is in most tokens,
    # the coldest in a handful
    assert int(counts.max()) >= 300 and int(counts.min()) * 20 <= int(counts.max())
    assert all(len(set(r.tolist())) == K for r in ids)   # distinct experts per token
    w = w4a16_random(E, H, I, seed=5)
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)
    h.store_awq_repack(*[t.to(cuda) for t in w], 128)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    y = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h)
    torch.cuda.synchronize()
    hot = int(counts.argmax())
    hot_tokens = [t for t in range(T) if hot in ids[t].tolist()][:4]
    s = token_sample(T, 20, seed=1, must=hot_tokens)
    assert max_rel_err(y.cpu()[s], _w4a16_oracle(x[s], ids[s], tw[s], w, E, I)) <= TOL
