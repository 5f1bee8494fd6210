"""Pins the oracle's Q8_0 quantizer and conversions with closed forms,
library routines and mathematical bounds (not by re-typing its formula).
Reference rule: Int8-gemm/gemm_kernels.cpp:25-58."""
import numpy as np
import pytest
import torch

import oracle
from helpers import bits


def test_zero_block():
    d, q = oracle.quantize_block_q8_0(np.zeros(32, np.float32))
    assert d == 0.0 and not q.any()


def test_exact_integers_scale_one():
    # amax = 127 -> d = 1, id = 1: integer inputs quantize to themselves
    x = np.arange(-15, 17, dtype=np.float32) * 4.0
    x[0] = -127.0
    d, q = oracle.quantize_block_q8_0(x)
    assert d == 1.0
    assert np.array_equal(q.astype(np.float32), x)


@pytest.mark.parametrize("p", [-6, -3, 0, 2, 5])
def test_power_of_two_scaling(p):
    # scaling by 2^p scales d by 2^p exactly and leaves q unchanged
    x = np.linspace(-127, 127, 32).round().astype(np.float32)
    d0, q0 = oracle.quantize_block_q8_0(x)
    d1, q1 = oracle.quantize_block_q8_0(x * np.float32(2.0 ** p))
    assert d1 == np.float32(d0 * 2.0 ** p)
    assert np.array_equal(q0, q1)


def test_ties_round_to_even():
    x = np.zeros(32, np.float32)
    x[0] = 127.0                       # d = 1
    x[1:9] = [0.5, 1.5, 2.5, 3.5, -0.5, -1.5, -2.5, -3.5]
    d, q = oracle.quantize_block_q8_0(x)
    assert d == 1.0
    assert list(q[1:9]) == [0, 2, 2, 4, 0, -2, -2, -4]


def test_amax_maps_to_127_and_error_bound():
    rng = np.random.default_rng(0)
    for _ in range(200):
        x = (rng.standard_normal(32) * rng.uniform(1e-3, 1e3)).astype(np.float32)
        d, q = oracle.quantize_block_q8_0(x)
        j = int(np.argmax(np.abs(x)))
        assert abs(int(q[j])) == 127 and np.sign(q[j]) == np.sign(x[j])
        assert d == np.float32(np.abs(x).max()) / np.float32(127.0)
        # round-to-nearest: |x - d q| <= d/2 (plus fp32 slack)
        err = np.abs(x.astype(np.float64) - float(d) * q.astype(np.float64))
        assert (err <= 0.5 * float(d) * (1 + 1e-5) + 1e-30).all()
        assert np.all((q == 0) | (np.sign(q) == np.sign(x)))


def test_act_quant_layout_bf16_fp16():
    rng = np.random.default_rng(1)
    T, H = 3, 256
    for dt, code in ((torch.bfloat16, 1), (torch.float16, 0)):
        x = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(dt)
        qs, d = oracle.quantize_act_q8_0(bits(x), code)
        xf = x.to(torch.float32).numpy().reshape(T, H // 32, 32)
        assert np.array_equal(d, np.abs(xf).max(-1) / np.float32(127.0))
        for t in range(T):
            for b in range(H // 32):
                d1, q1 = oracle.quantize_block_q8_0(xf[t, b])
                assert np.array_equal(qs[t, 32 * b:32 * b + 32], q1)


def test_weight_quant_fp16_scale():
    rng = np.random.default_rng(2)
    w = (rng.standard_normal((8, 128)) * 0.02).astype(np.float32)
    qs, d = oracle.quantize_weight_q8_0(w)
    amax = np.abs(w.reshape(8, 4, 32)).max(-1)
    d_expect = (amax / np.float32(127.0)).astype(np.float16).view(np.uint16)
    assert np.array_equal(d, d_expect)
    deq = qs.reshape(8, 4, 32).astype(np.float32) * d.view(np.float16).astype(np.float32)[..., None]
    assert np.abs(deq.reshape(8, 128) - w).max() <= 0.51 * amax.max() / 127 * 1.01


def test_f16_bf16_conversions_match_libraries():
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(4000) * 10 ** rng.uniform(-9, 6, 4000),
                           [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, -6e-8, 3e38]]).astype(np.float32)
    lib = oracle.lib()
    f16 = np.array([lib.orc_f32_to_f16(oracle.ctypes.c_float(v)) for v in vals], np.uint16)
    assert np.array_equal(f16, vals.astype(np.float16).view(np.uint16))
    bf = np.array([lib.orc_f32_to_bf16(oracle.ctypes.c_float(v)) for v in vals], np.uint16)
    tb = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bf, tb)
