"""GPU parity of the Q8_0 / Q4_0 path (the reference CPU algorithm,
Int8-gemm/q8_gemm.cpp:276-646) against the oracle on identical inputs.

* per-32-block int32 dot products: bit-exact (mi_moe_block_dots, the v_dot4
  routine of the lane-per-row kernels), Q8_0 and Q4_0, both projections;
* the int8-MFMA block routine of the grouped GEMMs (mi_moe_block_dots_mfma):
  its bias-accumulator int32 result and the first scaled product read back
  from it, bit-exact against the oracle's dots and (float)isum * dw, with
  extreme weights and activations;
* the fused layer: fp32 sums differ from the oracle only by the wave-split
  summation order, so outputs agree to max-rel-err <= 1e-2 (observed ~1e-3,
  dominated by rare intermediate Q8_0 rounding flips); above 96 (Q8_0) /
  160 (Q4_0) routed pairs the int8-MFMA grouped GEMMs run instead (k blocks
  summed in the reference's order), covered here by the (20, 10) and (200, 8)
  cases and the tile test; (12, 10) runs Q4_0 on the lane-per-row kernels and
  Q8_0 on the GEMMs;
* online Q8_0 weight quantization (quantize_and_store_expert) gives the same
  bytes as the oracle's quantize_weight_only restatement (checked through
  block dots) and the same layer output as the wire-format loader."""
import ctypes

import numpy as np
import pytest
import torch

import nanovllm_moe
import oracle
from helpers import bits, max_rel_err, topk_routing
import nanovllm_moe.formats as fmt

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _weights(qt, E, H, I, seed, sdt=torch.float16):
    g = torch.Generator().manual_seed(seed)
    if qt == 0:
        w13 = torch.randn(E, 2 * I, H, generator=g) * 0.05
        w2 = torch.randn(E, H, I, generator=g) * 0.05
        q13, d13 = oracle.quantize_weight_q8_0(w13.reshape(-1, H).numpy())
        q2, d2 = oracle.quantize_weight_q8_0(w2.reshape(-1, I).numpy())
        d13 = torch.from_numpy(d13.view(np.float16)).to(sdt).reshape(E, 2 * I, H // 32)
        d2 = torch.from_numpy(d2.view(np.float16)).to(sdt).reshape(E, H, I // 32)
        return (torch.from_numpy(q13.reshape(E, 2 * I, H)), d13,
                torch.from_numpy(q2.reshape(E, H, I)), d2, (w13, w2))
    q13, d13 = fmt.q4_0_random((E, 2 * I), H, generator=g, scale_dtype=sdt)
    q2, d2 = fmt.q4_0_random((E, H), I, generator=g, scale_dtype=sdt)
    return q13, d13, q2, d2, None


def _oracle(qt, x, ids, tw, w, E, I):
    q13, d13, q2, d2 = w[:4]
    acode = 1 if x.dtype == torch.bfloat16 else 0
    scode = 1 if d13.dtype == torch.bfloat16 else 0
    _, yf = oracle.moe_forward_q(qt, acode, scode, bits(x), tw.numpy(), ids.numpy(),
                                 q13.numpy(), bits(d13), q2.numpy(), bits(d2), E, I)
    return torch.from_numpy(yf)


def _handle(qt, E, H, I, w, on_device, cuda):
    h = torch.classes.nanovllm.MoEInfer(E, H, I, qt)
    ws = [t.to(cuda) for t in w[:4]] if on_device else list(w[:4])
    h.store_quantized_repack(*ws)
    return h


def _run(h, x, ids, tw, cuda):
    y = torch.ops.nanovllm.moe_forward(x.to(cuda), ids.to(cuda), tw.to(cuda), h)
    torch.cuda.synchronize()
    return y.cpu()


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T,K", [(1, 8), (5, 8), (12, 10), (20, 10), (40, 1), (200, 8)])
def test_forward_parity_small(cuda, qt, T, K):
    E, H, I = 16, 256, 128
    w = _weights(qt, E, H, I, seed=10 + qt)
    h = _handle(qt, E, H, I, w, T % 2 == 0, cuda)
    ids, tw = topk_routing(T, E, K, seed=T)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("T,K", [(150, 1), (70, 1), (16, 10)])
def test_ballot_routing_concentrated(cuda, qt, T, K):
    """Lane-per-row gate_up with the ballot routing over 2-3 batches of 64 ids
    (65-192 routed pairs), K = 1 with one expert taking more than 64 columns:
    Q4_0 at 150 / 70 / 160 pairs and Q8_0 at 70 pairs stay on the lane-per-row
    kernels (Q8_0 at 150 and 160 pairs takes the grouped GEMMs).  Three
    quarters of the tokens put their first pick on expert 3, and some ids are
    out of range."""
    E, H, I = 16, 256, 128
    w = _weights(qt, E, H, I, seed=20 + qt)
    h = _handle(qt, E, H, I, w, True, cuda)
    ids, tw = topk_routing(T, E, K, seed=T + K)
    ids = ids.clone()
    ids[: (3 * T) // 4, 0] = 3
    ids[T - 2, 0] = -1
    ids[T - 1, K - 1] = E
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
def test_forward_dtypes_and_invalid_ids(cuda, qt):
    E, H, I, T, K = 8, 192, 96, 6, 8
    w = _weights(qt, E, H, I, seed=3, sdt=torch.bfloat16)
    h = _handle(qt, E, H, I, w, True, cuda)
    ids, tw = topk_routing(T, E, K, seed=4)
    ids = ids.clone()
    ids[0, 2] = -1
    ids[1, :] = E + 3          # no valid id -> zeros
    ids[2, :] = 5              # one expert eight times
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(5)).to(torch.float16)
    y = _run(h, x, ids, tw, cuda)
    assert y.dtype == torch.float16
    assert torch.all(y[1] == 0)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
def test_one_launch_small_calls(cuda, qt):
    """The one-launch decode kernel at the sizes whose gate_up K is split over
    two workgroups (up to 12 routed pairs): one token with a duplicated
    expert and two out-of-range ids, one token with no valid id (zeros), one
    top-1 token and 12 top-1 tokens; every call against the oracle, and
    repeated calls (a new dispatch tag each) bit-identical."""
    E, H, I = 16, 256, 128
    w = _weights(qt, E, H, I, seed=70 + qt)
    h = _handle(qt, E, H, I, w, True, cuda)
    cases = []
    ids = torch.tensor([[3, 3, -1, 5, E, 7, 3, 0]], dtype=torch.int32)
    cases.append(ids)
    cases.append(torch.full((1, 8), E + 1, dtype=torch.int32))
    cases.append(torch.tensor([[9]], dtype=torch.int32))
    cases.append(topk_routing(12, E, 1, seed=71)[0])
    for i, ids in enumerate(cases):
        T, K = ids.shape
        tw = torch.softmax(torch.randn(T, K, generator=torch.Generator().manual_seed(i)), dim=-1)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(80 + i)).to(torch.bfloat16)
        y = _run(h, x, ids, tw, cuda)
        if bool((ids >= E).all() | (ids < 0).all()):
            assert torch.all(y == 0)
        assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL
        for _ in range(2):
            assert torch.equal(_run(h, x, ids, tw, cuda), y)


@pytest.mark.parametrize("qt", [0, 1])
def test_one_launch_graph_replay(cuda, qt):
    """Calls of 8 and 40 routed pairs (both forms of the one-launch kernel)
    captured in one HIP graph: every replay, with eager calls on the same
    handle between replays, equals the eager results bit for bit."""
    E, H, I = 16, 256, 128
    w = _weights(qt, E, H, I, seed=90 + qt)
    h = _handle(qt, E, H, I, w, True, cuda)
    cases = []
    for T, K, s in ((1, 8, 91), (5, 8, 92)):
        ids, tw = topk_routing(T, E, K, seed=s)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(s)).to(torch.bfloat16)
        cases.append((x.to(cuda), ids.to(cuda), tw.to(cuda)))
    outs = [torch.empty(x.shape[0], H, dtype=torch.bfloat16, device=cuda) for x, _, _ in cases]
    for (x, ids, tw), o in zip(cases, outs):
        torch.ops.nanovllm.moe_forward_out(x, ids, tw, h, o)
    torch.cuda.synchronize()
    eager = [o.cpu() for o in outs]
    for (x, ids, tw), e in zip(cases, eager):
        assert max_rel_err(e, _oracle(qt, x.cpu(), ids.cpu(), tw.cpu(), w, E, I)) <= TOL
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for (x, ids, tw), o in zip(cases, outs):
            torch.ops.nanovllm.moe_forward_out(x, ids, tw, h, o)
    for rep in range(3):
        for o in outs:
            o.zero_()
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o.cpu(), e), f"replay {rep}"
        x, ids, tw = cases[rep % 2]
        y = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), eager[rep % 2])


@pytest.mark.parametrize("qt", [0, 1])
def test_gemm_path_tiles_and_invalid_ids(cuda, qt):
    """Grouped-GEMM path: an expert with 64 + 64 + 2 rows (two full row tiles
    and a ragged one), one with 65, ids outside [0, E), fp16 activations and
    bf16 scales."""
    E, H, I, T, K = 8, 384, 256, 130, 8
    w = _weights(qt, E, H, I, seed=30 + qt, sdt=torch.bfloat16)
    h = _handle(qt, E, H, I, w, True, cuda)
    ids, tw = topk_routing(T, E, K, seed=31)
    ids = ids.clone()
    ids[:, 0] = 3                        # expert 3 in every token: 130 rows
    ids[:65, 1] = 6                      # expert 6 in 65 tokens (duplicates allowed)
    ids[0, 2] = -1
    ids[1, :] = E + 3                    # no valid id -> zeros
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(32)).to(torch.float16)
    y = _run(h, x, ids, tw, cuda)
    assert y.dtype == torch.float16
    assert torch.all(y[1] == 0)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
def test_gemm_many_rows_per_expert(cuda, qt):
    """Int8 GEMM row tiles of experts with 16 to 257 routed rows (a tile of
    64 rows is followed by a ragged one of 6, 36, 1 or 1 rows; 64 + 64 exact),
    ids outside [0, E), an expert absent."""
    E, H, I, T, K = 8, 256, 128, 90, 8          # 720 pairs >= 64 * E
    w = _weights(qt, E, H, I, seed=70 + qt, sdt=torch.bfloat16)
    h = _handle(qt, E, H, I, w, True, cuda)
    g = torch.Generator().manual_seed(71)
    ids = torch.full((T, K), 7, dtype=torch.int32)   # expert 7 absent unless written below
    flat = ids.view(-1)
    order = torch.randperm(T * K, generator=g)
    sizes = {0: 70, 1: 100, 2: 128, 3: 129, 4: 257, 5: 17, 6: 16}
    pos = 0
    for e, cnt in sizes.items():
        flat[order[pos:pos + cnt]] = e
        pos += cnt
    flat[order[pos:]] = -1                       # dropped pairs
    flat[order[pos]] = E + 5                     # out of range
    tw = torch.softmax(torch.randn(T, K, generator=g), dim=-1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(72)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("bs", [1, 8, 64])   # 64: 512 pairs, the int8 grouped-GEMM path
def test_qwen_shape(cuda, qt, bs):
    E, H, I = 128, 2048, 768
    w = _weights(qt, E, H, I, seed=99)
    h = _handle(qt, E, H, I, w, True, cuda)
    ids, tw = topk_routing(bs, E, 8, seed=bs)
    x = torch.randn(bs, H, generator=torch.Generator().manual_seed(bs)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


def _capi_handle(qt, E, H, I, w, cuda):
    L = nanovllm_moe.capi()
    hp = ctypes.c_void_p()
    nanovllm_moe.check(L.mi_moe_create(E, H, I, qt, ctypes.byref(hp)), "create")
    dev = [t.contiguous().to(cuda) for t in w[:4]]
    scode = 1 if w[1].dtype == torch.bfloat16 else 0
    nanovllm_moe.check(L.mi_moe_store_quantized(hp, *[ctypes.c_void_p(t.data_ptr()) for t in dev],
                                                 scode, 1, nanovllm_moe.stream_ptr()), "store")
    return L, hp


def _gpu_block_dots(L, hp, e, proj, a_qs, N, K, cuda):
    a = torch.from_numpy(a_qs).to(cuda)
    out = torch.empty(a_qs.shape[0], N, K // 32, dtype=torch.int32, device=cuda)
    nanovllm_moe.check(L.mi_moe_block_dots(hp, e, proj, ctypes.c_void_p(a.data_ptr()), a_qs.shape[0],
                                           ctypes.c_void_p(out.data_ptr()), nanovllm_moe.stream_ptr()),
                       "block_dots")
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("qt", [0, 1])
def test_block_dots_bit_exact(cuda, qt):
    E, H, I = 4, 256, 128
    w = _weights(qt, E, H, I, seed=21)
    L, hp = _capi_handle(qt, E, H, I, w, cuda)
    try:
        rng = np.random.default_rng(0)
        for e in (0, 3):
            for proj, (N, K, wq) in enumerate(((2 * I, H, w[0]), (H, I, w[2]))):
                a = rng.integers(-128, 128, size=(3, K)).astype(np.int8)
                a[0] = -128                                   # extreme magnitudes
                got = _gpu_block_dots(L, hp, e, proj, a, N, K, cuda)
                ref = oracle.block_dots(qt, a, wq[e].contiguous().numpy(), N, K)
                assert np.array_equal(got, ref)
    finally:
        L.mi_moe_destroy(hp)


def _extreme_wire(qt, E, H, I, seed):
    """Wire weights whose first rows hold the extremes: Q8_0 rows of -128, of
    127 and alternating; Q4_0 rows of nibble 0, of 15 and alternating; the
    rest uniform over the whole code range.  Scales: random fp16 of both
    signs, with a few large and tiny magnitudes."""
    rng = np.random.default_rng(seed)
    if qt == 0:
        q13 = rng.integers(-128, 128, size=(E, 2 * I, H)).astype(np.int8)
        q2 = rng.integers(-128, 128, size=(E, H, I)).astype(np.int8)
        for q in (q13, q2):
            q[:, 0] = -128
            q[:, 1] = 127
            q[:, 2, 0::2], q[:, 2, 1::2] = -128, 127
    else:
        def words(R, K):
            nib = rng.integers(0, 16, size=(E, R, K)).astype(np.uint32)
            nib[:, 0] = 0
            nib[:, 1] = 15
            nib[:, 2, 0::2], nib[:, 2, 1::2] = 0, 15
            w = np.zeros((E, R, K // 8), np.uint32)
            for i in range(8):
                w |= nib[:, :, i::8] << np.uint32(4 * i)
            return w.view(np.int32)
        q13, q2 = words(2 * I, H), words(H, I)

    def scales(shape):
        d = (rng.standard_normal(shape) * 0.01).astype(np.float16)
        d.reshape(-1)[:3] = np.array([60000.0, -1.0e-4, 6.1e-5], np.float16)
        return torch.from_numpy(d)
    return (torch.from_numpy(q13), scales((E, 2 * I, H // 32)), torch.from_numpy(q2), scales((E, H, I // 32)))


@pytest.mark.parametrize("qt", [0, 1])
def test_mfma_block_dots_bit_exact(cuda, qt):
    """The int8-MFMA block routine of the grouped GEMMs (mi_moe_block_dots_mfma)
    against the oracle's exact block dots: the MFMA result less its 1.5*2^23 bias
    is isum (Q4_0: 16*isum, nibbles entering as bytes 16*(n-8)), and the first
    scaled product read back from it as a float is the fp32 product
    (float)isum * dw of gemm_kernels.cpp:156-179 (Q4_0: 16 times it), bit for
    bit.  Activations include rows of -128, of 127 and alternating."""
    E, H, I = 2, 256, 128
    gq, gd, dq, dd = _extreme_wire(qt, E, H, I, seed=5 + qt)
    L = nanovllm_moe.capi()
    hp = ctypes.c_void_p()
    nanovllm_moe.check(L.mi_moe_create(E, H, I, qt, ctypes.byref(hp)), "create")
    try:
        nanovllm_moe.check(L.mi_moe_store_quantized(hp, gq.data_ptr(), gd.data_ptr(), dq.data_ptr(),
                                                    dd.data_ptr(), nanovllm_moe.F16, 0, None), "store")
        rng = np.random.default_rng(11)
        for e in range(E):
            for proj, (N, K, wq, wd) in enumerate(((2 * I, H, gq, gd), (H, I, dq, dd))):
                a = rng.integers(-128, 128, size=(19, K)).astype(np.int8)
                a[0], a[1] = -128, 127
                a[2, 0::2], a[2, 1::2] = -128, 127
                at = torch.from_numpy(a).to(cuda)
                acc = torch.empty(a.shape[0], N, K // 32, dtype=torch.int32, device=cuda)
                prod = torch.empty(a.shape[0], N, K // 32, dtype=torch.float32, device=cuda)
                nanovllm_moe.check(L.mi_moe_block_dots_mfma(hp, e, proj, at.data_ptr(), a.shape[0],
                                                            acc.data_ptr(), prod.data_ptr(),
                                                            nanovllm_moe.stream_ptr()), "block_dots_mfma")
                torch.cuda.synchronize()
                isum = oracle.block_dots(qt, a, wq[e].contiguous().numpy(), N, K)
                dw = wd[e].numpy().astype(np.float32)[None, :, :]
                want = isum.astype(np.float32) * dw             # fp32 RNE product, as the reference
                m = 16 if qt == 1 else 1
                got_acc, got_prod = acc.cpu().numpy(), prod.cpu().numpy()
                assert np.array_equal(got_acc, isum * m), (e, proj)
                want = want * np.float32(m)
                # bit for bit, except the sign of a zero product: the fma gives +0 where
                # (float)0 * dw is -0 (dw < 0); a zero addend of either sign leaves the
                # reference's running sum, which starts at +0, unchanged
                nz = want != 0
                assert np.array_equal(got_prod.view(np.uint32)[nz], want.view(np.uint32)[nz]), (e, proj)
                assert np.all(got_prod[~nz] == 0), (e, proj)
                if qt == 0:   # the extremes reach the block's largest |isum|
                    assert np.abs(isum).max() == 32 * 128 * 128
    finally:
        L.mi_moe_destroy(hp)


def test_online_quant_matches_oracle(cuda):
    E, H, I = 8, 256, 128
    w = _weights(0, E, H, I, seed=31)
    w13, w2 = w[4]
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 0)
    for e in range(E):
        h.quantize_and_store_expert(e, "gate_proj", w13[e, :I].contiguous())
        h.quantize_and_store_expert(e, "up_proj", w13[e, I:].contiguous().to(cuda))
        h.quantize_and_store_expert(e, "down_proj", w2[e].contiguous())
    T, K = 7, 8
    ids, tw = topk_routing(T, E, K, seed=2)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    h2 = _handle(0, E, H, I, w, False, cuda)
    y2 = _run(h2, x, ids, tw, cuda)
    assert torch.equal(y, y2)          # same bytes, same scales, same kernels
    assert max_rel_err(y, _oracle(0, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
@pytest.mark.parametrize("E,H,I,T,K", [(8, 5120, 256, 1, 8), (8, 5120, 256, 5, 1), (8, 5120, 256, 9, 8),
                                       (8, 256, 14336, 1, 8), (8, 256, 14336, 30, 1)])
def test_large_shape_parity(cuda, qt, E, H, I, T, K):
    """GLM-like H = 5120 (the lane-per-row gate_up needs 10H + 16 KB of LDS) and
    Mixtral-like I = 14336 (the token-major down kernel needs about 18 KB per
    routed expert, the expert-major one 10I + 16 KB): calls of up to 64 routed
    pairs take the lane-per-row kernels where their LDS fits the device and the
    int8 grouped GEMMs otherwise.  top_k 1 and 8, as the reference's routing
    accepts (Int8-gemm/moe_common.cpp:197-215)."""
    w = _weights(qt, E, H, I, seed=60 + qt)
    h = _handle(qt, E, H, I, w, True, cuda)
    ids, tw = topk_routing(T, E, K, seed=T + 1)
    x = torch.randn(T, H, generator=torch.Generator().manual_seed(T + 2)).to(torch.bfloat16)
    y = _run(h, x, ids, tw, cuda)
    assert max_rel_err(y, _oracle(qt, x, ids, tw, w, E, I)) <= TOL


@pytest.mark.parametrize("qt", [0, 1])
def test_cpu_and_hip_keys_agree(cuda, qt, monkeypatch):
    """One handle with both copies (MIMOE_HOST_WEIGHTS=1): the CPU key (the
    reference algorithm on host cores) and the HIP key agree to the parity
    tolerance on the Qwen3 shape at the reference benchmark's decode sizes."""
    monkeypatch.setenv("MIMOE_HOST_WEIGHTS", "1")
    E, H, I = 128, 2048, 768
    w = _weights(qt, E, H, I, seed=17)
    h = _handle(qt, E, H, I, w, False, cuda)
    for T in (1, 4):
        ids, tw = topk_routing(T, E, 8, seed=40 + T)
        x = torch.randn(T, H, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16)
        y_cpu = torch.ops.nanovllm.moe_forward(x, ids, tw, h)
        y_gpu = _run(h, x, ids, tw, cuda)
        assert y_cpu.device.type == "cpu"
        assert max_rel_err(y_gpu, y_cpu) <= TOL
        assert max_rel_err(y_cpu, _oracle(qt, x, ids, tw, w, E, I)) <= TOL
