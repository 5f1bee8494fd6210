"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py
from a numpy restatement independent of the oracle and the kernels).

CPU: the oracle reproduces every fixture (bit-exact for Q8_0 bytes, routing
and block dots; within 1e-5 of the float64 W4A16 output).  GPU: the HIP path,
called through the C ABI / the torch op, reproduces the same fixtures
(bit-exact for the integer parts; W4A16 output within the 1e-2 parity
tolerance, the gap being the bf16 rounding of the intermediate activation and
of the output)."""
import ctypes
import os

import numpy as np
import pytest
import torch

import nanovllm_moe
import oracle
from helpers import max_rel_err

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


# ---------------------------------------------------------------- CPU (oracle)
def test_q8_0_fixture_oracle():
    g = _load("golden_q8_0.npz")
    for b in range(g["x"].shape[0]):
        d, qs = oracle.quantize_block_q8_0(g["x"][b])
        assert np.array_equal(qs, g["qs"][b]), b
        assert np.float32(d).view(np.uint32) == g["d"][b].view(np.uint32), b
    # the activation-level entry point over the same values laid out [T, H]
    bits = g["x_bf16_bits"].reshape(8, -1)
    q, d = oracle.quantize_act_q8_0(bits, 1)
    assert np.array_equal(q.reshape(-1, 32), g["qs"])
    assert np.array_equal(d.reshape(-1).view(np.uint32), g["d"].view(np.uint32))


def test_route_fixture_oracle():
    g = _load("golden_route.npz")
    counts, starts, tmap, scat = oracle.route(g["ids"], int(g["E"]))
    assert np.array_equal(counts, g["counts"])
    assert np.array_equal(starts, g["starts"])
    assert np.array_equal(tmap, g["token_map"])
    assert np.array_equal(scat, g["scatter"])


def test_q4_dots_fixture_oracle():
    g = _load("golden_q4_dots.npz")
    N, K = g["w_words"].shape[0], g["a_qs"].shape[1]
    got = oracle.block_dots(1, g["a_qs"], g["w_words"], N, K)
    assert np.array_equal(got, g["isum"])


def test_w4a16_fixture_oracle():
    g = _load("golden_w4a16.npz")
    _, yf = oracle.moe_forward_w4a16(1, 1, g["x_bf16_bits"], g["topk_w"], g["topk_ids"], g["w13_q"],
                                     g["w13_z"], g["w13_s_bf16"], g["w2_q"], g["w2_z"], g["w2_s_bf16"],
                                     int(g["E"]), int(g["I"]), int(g["group"]))
    assert max_rel_err(torch.from_numpy(yf), torch.from_numpy(g["y"])) <= 1e-5


# ---------------------------------------------------------------- GPU (HIP path)
@pytest.mark.gpu
def test_q8_0_fixture_gpu(cuda):
    g = _load("golden_q8_0.npz")
    bits = torch.from_numpy(g["x_bf16_bits"].reshape(8, -1).view(np.int16)).to(cuda)
    T, H = bits.shape
    qs = torch.empty(T, H, dtype=torch.int8, device=cuda)
    d = torch.empty(T, H // 32, dtype=torch.float32, device=cuda)
    L = nanovllm_moe.capi()
    nanovllm_moe.check(L.mi_moe_quantize_act_q8_0(_ptr(bits), 1, T, H, _ptr(qs), _ptr(d),
                                                  nanovllm_moe.stream_ptr()), "quantize_act")
    torch.cuda.synchronize()
    assert np.array_equal(qs.cpu().numpy().reshape(-1, 32), g["qs"])
    assert np.array_equal(d.cpu().numpy().reshape(-1).view(np.uint32), g["d"].view(np.uint32))


@pytest.mark.gpu
def test_route_fixture_gpu(cuda):
    g = _load("golden_route.npz")
    ids = torch.from_numpy(g["ids"]).to(cuda)
    T, K = ids.shape
    E = int(g["E"])
    counts = torch.full((E,), -7, dtype=torch.int32, device=cuda)
    starts = torch.full((E + 1,), -7, dtype=torch.int32, device=cuda)
    tmap = torch.full((T * K,), -7, dtype=torch.int32, device=cuda)
    scat = torch.full((T * K,), -7, dtype=torch.int32, device=cuda)
    L = nanovllm_moe.capi()
    nanovllm_moe.check(L.mi_moe_route(_ptr(ids), T, K, E, _ptr(counts), _ptr(starts), _ptr(tmap),
                                      _ptr(scat), nanovllm_moe.stream_ptr()), "route")
    torch.cuda.synchronize()
    assert np.array_equal(counts.cpu().numpy(), g["counts"])
    assert np.array_equal(starts.cpu().numpy(), g["starts"])
    nv = int(g["starts"][E])
    assert np.array_equal(tmap.cpu().numpy()[:nv], g["token_map"][:, 0])
    assert np.array_equal(scat.cpu().numpy().reshape(T, K), g["scatter"])


@pytest.mark.gpu
def test_q4_dots_fixture_gpu(cuda):
    """The fixture's 64 rows x 128 k are the gate_up rows of a one-expert
    Q4_0 handle (H = 128, I = 32)."""
    g = _load("golden_q4_dots.npz")
    H, I = 128, 32
    L = nanovllm_moe.capi()
    hp = ctypes.c_void_p()
    nanovllm_moe.check(L.mi_moe_create(1, H, I, 1, ctypes.byref(hp)), "create")
    try:
        gu = torch.from_numpy(g["w_words"].reshape(1, 2 * I, H // 8)).to(cuda)
        gu_d = torch.ones(1, 2 * I, H // 32, dtype=torch.float16, device=cuda)
        dn = torch.zeros(1, H, I // 8, dtype=torch.int32, device=cuda)
        dn_d = torch.ones(1, H, I // 32, dtype=torch.float16, device=cuda)
        nanovllm_moe.check(L.mi_moe_store_quantized(hp, _ptr(gu), _ptr(gu_d), _ptr(dn), _ptr(dn_d),
                                                    0, 1, nanovllm_moe.stream_ptr()), "store")
        a = torch.from_numpy(g["a_qs"]).to(cuda)
        out = torch.empty(a.shape[0], 2 * I, H // 32, dtype=torch.int32, device=cuda)
        nanovllm_moe.check(L.mi_moe_block_dots(hp, 0, 0, _ptr(a), a.shape[0], _ptr(out),
                                               nanovllm_moe.stream_ptr()), "block_dots")
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), g["isum"])
    finally:
        L.mi_moe_destroy(hp)


@pytest.mark.gpu
def test_w4a16_fixture_gpu(cuda):
    g = _load("golden_w4a16.npz")
    E, H, I, grp = int(g["E"]), int(g["H"]), int(g["I"]), int(g["group"])
    h = torch.classes.nanovllm.MoEInfer(E, H, I, 2)

    def bf16(a):
        return torch.from_numpy(a.view(np.int16)).view(torch.bfloat16)

    h.store_awq_repack(torch.from_numpy(g["w13_q"]), torch.from_numpy(g["w13_z"]), bf16(g["w13_s_bf16"]),
                       torch.from_numpy(g["w2_q"]), torch.from_numpy(g["w2_z"]), bf16(g["w2_s_bf16"]), grp)
    x = bf16(g["x_bf16_bits"]).to(cuda)
    y = torch.ops.nanovllm.moe_forward(x, torch.from_numpy(g["topk_ids"]).to(cuda),
                                       torch.from_numpy(g["topk_w"]).to(cuda), h)
    torch.cuda.synchronize()
    assert max_rel_err(y.cpu(), torch.from_numpy(g["y"])) <= 1e-2
