"""Pins the oracle's fused forward (Int8-gemm/q8_gemm.cpp:276-646) and the
W4A16 restatement against dense float64 torch formulas, which restate the
reference's own check reference_moe_fp16 (Int8-gemm/test/fused_moe_cpu.py:
40-95) in float64 over the dequantized weights.  The matrix-product form is
independent of the oracle's per-block loops, so a transposed operand, a
swapped gate/up half, a wrong scale index or a wrong combine weight fails."""
import numpy as np
import pytest
import torch

import oracle
import nanovllm_moe.formats as fmt
from helpers import bits, topk_routing, max_rel_err, w4a16_random


def _silu_mul64(gu, I):
    g, u = gu[..., :I], gu[..., I:]
    return u * (g / (1.0 + np.exp(-g)))


def _dense_q(qt, x_bits, act_code, ids, tw, gu_qs, gu_d, dn_qs, dn_d, sdt, E, H, I):
    """float64 dense restatement with the same two quantization points."""
    xq, xd = oracle.quantize_act_q8_0(x_bits, act_code)
    xdeq = xq.astype(np.float64).reshape(-1, H // 32, 32) * xd.astype(np.float64)[..., None]
    xdeq = xdeq.reshape(-1, H)
    gu_qs_t, dn_qs_t = torch.from_numpy(gu_qs), torch.from_numpy(dn_qs)
    if qt == 0:
        W13 = fmt.q8_0_dequant(gu_qs_t, gu_d).double().numpy()
        W2 = fmt.q8_0_dequant(dn_qs_t, dn_d).double().numpy()
    else:
        W13 = fmt.q4_0_dequant(gu_qs_t, gu_d).double().numpy()
        W2 = fmt.q4_0_dequant(dn_qs_t, dn_d).double().numpy()
    T, K = ids.shape
    y = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            e = ids[t, k]
            if not (0 <= e < E):
                continue
            gu = W13[e] @ xdeq[t]
            act = _silu_mul64(gu, I).astype(np.float32)
            aq = np.zeros(I, np.int8)
            ad = np.zeros(I // 32, np.float32)
            for b in range(I // 32):
                ad[b], aq[32 * b:32 * b + 32] = oracle.quantize_block_q8_0(act[32 * b:32 * b + 32])
            adeq = (aq.astype(np.float64).reshape(-1, 32) * ad.astype(np.float64)[:, None]).reshape(I)
            y[t] += float(tw[t, k]) * (W2[e] @ adeq)
    return y


def _q_weights(qt, E, H, I, seed, sdt):
    g = torch.Generator().manual_seed(seed)
    if qt == 0:
        w13 = torch.randn(E, 2 * I, H, generator=g) * 0.05
        w2 = torch.randn(E, H, I, generator=g) * 0.05
        q13, d13 = oracle.quantize_weight_q8_0(w13.reshape(-1, H).numpy())
        q2, d2 = oracle.quantize_weight_q8_0(w2.reshape(-1, I).numpy())
        d13 = torch.from_numpy(d13.view(np.float16)).to(sdt)
        d2 = torch.from_numpy(d2.view(np.float16)).to(sdt)
        return q13.reshape(E, 2 * I, H), d13.reshape(E, 2 * I, H // 32), q2.reshape(E, H, I), d2.reshape(E, H, I // 32)
    q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g, scale_dtype=sdt)
    q2, d2 = fmt.q4_0_random((E, H), I, generator=g, scale_dtype=sdt)
    return q13.numpy(), d13, q2.numpy(), d2


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("adt,sdt", [(torch.bfloat16, torch.float16), (torch.float16, torch.bfloat16)])
def test_forward_q_vs_dense(qt, adt, sdt):
    E, H, I, T, K = 8, 256, 128, 6, 8
    gu_qs, gu_d, dn_qs, dn_d = _q_weights(qt, E, H, I, 10 + qt, sdt)
    ids, tw = topk_routing(T, E, K, seed=3)
    ids = ids.numpy().copy()
    ids[1, 2] = -1          # dropped ids
    ids[2, :] = E + 5       # a token with no valid id -> zero row
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(4)).to(adt)
    acode = 1 if adt == torch.bfloat16 else 0
    scode = 1 if sdt == torch.bfloat16 else 0
    y, yf = oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids, gu_qs, bits(gu_d),
                                 dn_qs, bits(dn_d), E, I, tp=1)
    dense = _dense_q(qt, bits(x), acode, ids, tw.numpy(), gu_qs, gu_d, dn_qs, dn_d, sdt, E, H, I)
    assert np.all(yf[2] == 0) and np.all(y[2] == 0)
    assert max_rel_err(torch.from_numpy(yf), torch.from_numpy(dense)) < 2e-3
    # tp=2 only reorders fp32 sums (Int8-gemm/q8_gemm.cpp:621-641)
    _, yf2 = oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids, gu_qs, bits(gu_d),
                                  dn_qs, bits(dn_d), E, I, tp=2)
    assert max_rel_err(torch.from_numpy(yf2), torch.from_numpy(yf)) < 1e-5
    # the cast is RNE of the fp32 value
    ref_cast = torch.from_numpy(yf).to(adt)
    assert np.array_equal(y, bits(ref_cast))


def test_forward_q_unsupported_topk_and_all_invalid():
    E, H, I = 4, 64, 32
    gu_qs, gu_d, dn_qs, dn_d = _q_weights(0, E, H, I, 1, torch.float16)
    x = torch.randn(2, H).to(torch.bfloat16)
    with pytest.raises(RuntimeError):
        oracle.moe_forward_q(0, 1, 0, bits(x), np.ones((2, 3), np.float32), np.zeros((2, 3), np.int32),
                             gu_qs, bits(gu_d), dn_qs, bits(dn_d), E, I)
    y, yf = oracle.moe_forward_q(0, 1, 0, bits(x), np.ones((2, 1), np.float32), np.full((2, 1), -1, np.int32),
                                 gu_qs, bits(gu_d), dn_qs, bits(dn_d), E, I)
    assert not y.any() and not yf.any()


def test_reference_own_fp16_check_q4():
    """The reference's accuracy check (Int8-gemm/test/fused_moe_cpu_int4.py:
    135-173, 287-289): rel-RMSE vs an fp16 dense model of the Q4_0 weights
    below 0.1."""
    E, H, I, T, K = 8, 256, 128, 8, 8
    gu_qs, gu_d, dn_qs, dn_d = _q_weights(1, E, H, I, 7, torch.float16)
    W13 = fmt.q4_0_dequant(torch.from_numpy(gu_qs), gu_d).to(torch.float16)
    W2 = fmt.q4_0_dequant(torch.from_numpy(dn_qs), dn_d).to(torch.float16)
    ids, tw = topk_routing(T, E, K, seed=8)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(9)).to(torch.float16)
    out = torch.zeros(T, H)
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            gate = (x[t].float() @ W13[e, :I].float().t()).half()
            up = (x[t].float() @ W13[e, I:].float().t()).half()
            act = (torch.nn.functional.silu(gate.float()) * up.float()).half()
            ye = (act.float() @ W2[e].float().t()).half()
            out[t] += ye.float() * tw[t, k]
    y, _ = oracle.moe_forward_q(1, 0, 0, bits(x), tw.numpy(), ids.numpy(), gu_qs, bits(gu_d),
                                dn_qs, bits(dn_d), E, I)
    yv = torch.from_numpy(y.view(np.float16)).float()
    rel_rmse = float(torch.sqrt(((yv - out) ** 2).mean()) / torch.sqrt((out ** 2).mean()))
    assert rel_rmse < 0.1


def test_expf_and_silu():
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.uniform(-87, 88, 3000), rng.uniform(-3, 3, 3000), [0.0, -0.0, 1.0, -1.0]]).astype(np.float32)
    got = oracle.expf_vec(xs).astype(np.float64)
    ref = np.exp(xs.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - ref) <= 2 * ulp).all()
    assert oracle.expf(0.0) == 1.0
    assert oracle.expf(100.0) == float("inf") and oracle.expf(-100.0) == 0.0
    row = rng.standard_normal(64).astype(np.float32) * 4
    out = oracle.silu_and_mul(row)
    ref = _silu_mul64(row.astype(np.float64), 32)
    assert np.allclose(out, ref, rtol=2e-6, atol=1e-7)


def test_awq_known_answer_and_roundtrip():
    # slot s of word 0 holds value s -> column AWQ_ORDER[s] gets value s
    K, N = 128, 8
    qw = np.zeros((K, 1), np.int32)
    qw[:] = np.int32(0x76543210)
    qz = np.zeros((1, 1), np.int32)
    s = torch.ones(1, N, dtype=torch.bfloat16)
    w = oracle.awq_dequant(qw, qz, bits(s), 1, 128)
    for slot, col in enumerate(fmt.AWQ_ORDER):
        assert (w[col] == slot).all()
    q = torch.randint(0, 16, (3, 64, 40))
    assert torch.equal(fmt.awq_unpack(fmt.awq_pack(q)), q)


def test_forward_w4a16_vs_dense():
    E, H, I, T, K = 6, 256, 256, 5, 4
    w13_q, w13_z, w13_s, w2_q, w2_z, w2_s = w4a16_random(E, H, I, seed=11)
    ids, tw = topk_routing(T, E, K, seed=12)
    ids = ids.clone()
    ids[3, 1] = -1
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(13)).to(torch.bfloat16)
    y, yf = oracle.moe_forward_w4a16(1, 1, bits(x), tw.numpy(), ids.numpy(), w13_q.numpy(),
                                     w13_z.numpy(), bits(w13_s), w2_q.numpy(), w2_z.numpy(),
                                     bits(w2_s), E, I)
    W13 = fmt.awq_dequant(w13_q, w13_z, w13_s).double()      # [E, 2I, H]
    W2 = fmt.awq_dequant(w2_q, w2_z, w2_s).double()          # [E, H, I]
    xd = x.double()
    dense = torch.zeros(T, H, dtype=torch.float64)
    for t in range(T):
        for k in range(K):
            e = int(ids[t, k])
            if e < 0:
                continue
            gu = W13[e] @ xd[t]
            act = gu[I:] * (gu[:I] / (1 + torch.exp(-gu[:I])))
            dense[t] += float(tw[t, k]) * (W2[e] @ act)
    assert max_rel_err(torch.from_numpy(yf), dense) < 1e-5
    assert np.array_equal(y, bits(torch.from_numpy(yf).to(torch.bfloat16)))
