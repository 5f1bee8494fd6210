"""Wire formats accepted by the MoE handle, and producers for them.

Formats (all per expert, stacked on a leading E axis):

* Q8_0 -- ``store_quantized_repack`` of the reference
  (Int8-gemm/moe_infer.cpp:96-282): ``gate_up_qs`` int8 [E,2I,H] (rows [0,I)
  gate_proj, [I,2I) up_proj), ``gate_up_d`` fp16/bf16 [E,2I,H/32],
  ``down_qs`` int8 [E,H,I], ``down_d`` [E,H,I/32].
* Q4_0 -- same, with ``*_qs`` int32/uint32 [E,2I,H/8] and [E,H,I/8]; element
  k of a row is nibble k%8 (bits 4(k%8)..) of word k/8 and its value is
  ``nibble - 8`` (Int8-gemm/gemm_kernels.cpp:542,
  Int8-gemm/test/fused_moe_cpu_int4.py:58-71).
* W4A16 (AWQ layout, build-defined: the reference's W4A16 loader lives in an
  absent submodule) -- ``w13_qweight`` int32 [E,H,2I/8], ``w13_qzeros`` int32
  [E,H/g,2I/8], ``w13_scales`` [E,H/g,2I]; ``w2_qweight`` int32 [E,I,H/8],
  ``w2_qzeros`` [E,I/g,H/8], ``w2_scales`` [E,I/g,H].  Output columns are packed
  8 per int32 with nibble slot s holding column ``8j + AWQ_ORDER[s]``.
  Dequantized weight: ``W[n,k] = (q[k,n] - z[k//g,n]) * s[k//g,n]``.

All producers are plain torch and run on any device.
"""
from __future__ import annotations

import torch

AWQ_ORDER = (0, 2, 4, 6, 1, 3, 5, 7)


def _to_i32_wrap(v: torch.Tensor) -> torch.Tensor:
    """int64 tensor holding uint32 values -> int32 with two's-complement wrap."""
    v = v & 0xFFFFFFFF
    return torch.where(v >= 2**31, v - 2**32, v).to(torch.int32)


def awq_pack(q: torch.Tensor) -> torch.Tensor:
    """q: integer tensor [..., N] with values 0..15 -> int32 [..., N/8] (AWQ order)."""
    *lead, n = q.shape
    assert n % 8 == 0
    q = q.to(torch.int64).reshape(*lead, n // 8, 8)
    out = torch.zeros(*lead, n // 8, dtype=torch.int64, device=q.device)
    for slot, col in enumerate(AWQ_ORDER):
        out |= q[..., col] << (4 * slot)
    return _to_i32_wrap(out)


def awq_unpack(packed: torch.Tensor) -> torch.Tensor:
    """int32 [..., N/8] -> int64 [..., N] nibble values (inverse of awq_pack)."""
    p = packed.to(torch.int64) & 0xFFFFFFFF
    *lead, n8 = p.shape
    out = torch.empty(*lead, n8, 8, dtype=torch.int64, device=p.device)
    for slot, col in enumerate(AWQ_ORDER):
        out[..., col] = (p >> (4 * slot)) & 0xF
    return out.reshape(*lead, n8 * 8)


def awq_quantize(w: torch.Tensor, group: int = 128, scale_dtype=torch.bfloat16):
    """Asymmetric 4-bit quantization of fp weights along K (the input dim).

    w: [..., N, K] (output-major, like nn.Linear.weight).  Per (n, group of
    ``group`` k): s = (max-min)/15 rounded to ``scale_dtype``,
    z = clamp(RNE(-min/s), 0, 15), q = clamp(RNE(w/s) + z, 0, 15).
    Returns AWQ tensors (qweight [..., K, N/8], qzeros [..., K/g, N/8],
    scales [..., K/g, N]).
    """
    *lead, N, K = w.shape
    assert K % group == 0 and N % 8 == 0
    wg = w.to(torch.float32).reshape(*lead, N, K // group, group)
    mn = wg.amin(dim=-1)
    mx = wg.amax(dim=-1)
    s = ((mx - mn) / 15.0).to(scale_dtype)
    sf = s.to(torch.float32)
    sf = torch.where(sf == 0, torch.ones_like(sf), sf)
    z = torch.clamp(torch.round(-mn / sf), 0, 15)
    q = torch.clamp(torch.round(wg / sf.unsqueeze(-1)) + z.unsqueeze(-1), 0, 15)
    q = q.reshape(*lead, N, K).transpose(-1, -2).contiguous()         # [..., K, N]
    qweight = awq_pack(q)
    qzeros = awq_pack(z.transpose(-1, -2).contiguous())                # [..., K/g, N/8]
    scales = torch.where(s.to(torch.float32) == 0, torch.ones_like(sf), s.to(torch.float32))
    scales = scales.to(scale_dtype).transpose(-1, -2).contiguous()     # [..., K/g, N]
    return qweight, qzeros, scales


def awq_dequant(qweight, qzeros, scales, group: int = 128) -> torch.Tensor:
    """AWQ tensors -> fp32 weights [..., N, K]."""
    q = awq_unpack(qweight).to(torch.float32)                 # [..., K, N]
    z = awq_unpack(qzeros).to(torch.float32)                  # [..., K/g, N]
    s = scales.to(torch.float32)
    z = z.repeat_interleave(group, dim=-2)
    s = s.repeat_interleave(group, dim=-2)
    return ((q - z) * s).transpose(-1, -2).contiguous()


def q4_0_unpack(qs: torch.Tensor) -> torch.Tensor:
    """Q4_0 wire words [..., K/8] -> int64 values nibble-8 [..., K] (sequential nibbles)."""
    p = qs.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, device=p.device, dtype=torch.int64) * 4
    v = (p.unsqueeze(-1) >> shifts) & 0xF
    return v.reshape(*qs.shape[:-1], qs.shape[-1] * 8) - 8


def q4_0_pack(vals: torch.Tensor) -> torch.Tensor:
    """int values in [-8,7] [..., K] -> Q4_0 wire int32 words [..., K/8]."""
    *lead, k = vals.shape
    n = (vals.to(torch.int64) + 8).reshape(*lead, k // 8, 8)
    shifts = torch.arange(8, device=n.device, dtype=torch.int64) * 4
    return _to_i32_wrap((n << shifts).sum(dim=-1))


def q4_0_quantize(w: torch.Tensor, scale_dtype=torch.float16):
    """Symmetric Q4_0 along K, 32 per block: d = amax/7 (stored in scale_dtype),
    q = clamp(RNE(w/d), -8, 7).  Returns (qs int32 [...,K/8], d [...,K/32])."""
    *lead, K = w.shape
    wb = w.to(torch.float32).reshape(*lead, K // 32, 32)
    d = (wb.abs().amax(dim=-1) / 7.0).to(scale_dtype)
    df = d.to(torch.float32)
    inv = torch.where(df == 0, torch.zeros_like(df), 1.0 / torch.where(df == 0, torch.ones_like(df), df))
    q = torch.clamp(torch.round(wb * inv.unsqueeze(-1)), -8, 7).reshape(*lead, K)
    return q4_0_pack(q), d


def q4_0_random(shape_rows, K: int, generator=None, device="cpu", scale_dtype=torch.float16):
    """The reference generator's recipe (Int8-gemm/test/fused_moe_cpu_int4.py:74-115):
    uniform random nibbles, d = U[0,1) * (1/8) * sqrt(1/K)."""
    nwords = K // 8
    words = torch.randint(0, 2**32, (*shape_rows, nwords), generator=generator,
                          dtype=torch.int64, device=device)
    d = (torch.rand((*shape_rows, K // 32), generator=generator, device=device)
         * (1.0 / 8) * (1.0 / K) ** 0.5).to(scale_dtype)
    return _to_i32_wrap(words), d


def q8_0_dequant(qs: torch.Tensor, d: torch.Tensor) -> torch.Tensor:
    """Q8_0 wire [..., K] int8 + d [..., K/32] -> fp32 [..., K]."""
    return (qs.to(torch.float32).reshape(*qs.shape[:-1], -1, 32)
            * d.to(torch.float32).unsqueeze(-1)).reshape(qs.shape)


def q4_0_dequant(qs: torch.Tensor, d: torch.Tensor) -> torch.Tensor:
    v = q4_0_unpack(qs).to(torch.float32)
    return (v.reshape(*v.shape[:-1], -1, 32) * d.to(torch.float32).unsqueeze(-1)).reshape(v.shape)


def bytes_per_expert(quant: int, H: int, I: int, group: int = 128) -> int:
    """Algorithmic weight bytes per expert (3*H*I parameters)."""
    n = 3 * H * I
    if quant == 0:      # Q8_0: int8 + fp16 d per 32
        return n + n // 32 * 2
    if quant == 1:      # Q4_0: 4-bit + fp16 d per 32
        return n // 2 + n // 32 * 2
    # W4A16: 4-bit + 2-byte scale + 4-bit zero per group
    return n // 2 + n // group * 2 + n // group // 2
