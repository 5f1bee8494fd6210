"""Shared synthetic-data helpers for the tests (seeded, numpy/torch only)."""
import numpy as np
import torch

import nanovllm_moe.formats as fmt


def bits(t: torch.Tensor) -> np.ndarray:
    """fp16/bf16 tensor -> numpy uint16 raw bits."""
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, dtype) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype)


def topk_routing(T, E, K, seed, device="cpu"):
    """N(0,1) logits -> top-k (sorted) -> softmax over the k values
    (make_topk_from_logits_cpu, Int8-gemm/test/fused_moe_cpu.py:20-37)."""
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E, generator=g)
    val, ids = torch.topk(logits, K, dim=-1, largest=True, sorted=True)
    w = torch.softmax(val, dim=-1)
    return ids.to(torch.int32).contiguous(), w.to(torch.float32).contiguous()


def w4a16_random(E, H, I, seed, scale_dtype=torch.bfloat16, group=128):
    """Random AWQ tensors (uniform nibbles/zeros, scales ~ 0.02/7)."""
    g = torch.Generator().manual_seed(seed)
    def rint32(*shape):
        v = torch.randint(0, 2**32, shape, generator=g, dtype=torch.int64)
        return torch.where(v >= 2**31, v - 2**32, v).to(torch.int32)
    w13_q = rint32(E, H, 2 * I // 8)
    w13_z = rint32(E, H // group, 2 * I // 8)
    w13_s = (torch.rand(E, H // group, 2 * I, generator=g) * 0.004 + 0.001).to(scale_dtype)
    w2_q = rint32(E, I, H // 8)
    w2_z = rint32(E, I // group, H // 8)
    w2_s = (torch.rand(E, I // group, H, generator=g) * 0.004 + 0.001).to(scale_dtype)
    return w13_q, w13_z, w13_s, w2_q, w2_z, w2_s


def w4a16_from_normal(E, H, I, seed, scale_dtype=torch.bfloat16, group=128, std=0.02, device="cpu"):
    """The BASELINE recipe: fp weights ~ N(0, std^2) quantized AWQ-style (on
    `device`; the wire tensors are returned on the CPU)."""
    g = torch.Generator(device=device).manual_seed(seed)
    w1 = torch.randn(E, 2 * I, H, generator=g, device=device) * std
    a = [t.cpu() for t in fmt.awq_quantize(w1, group, scale_dtype)]
    del w1
    w2 = torch.randn(E, H, I, generator=g, device=device) * std
    b = [t.cpu() for t in fmt.awq_quantize(w2, group, scale_dtype)]
    return a[0], a[1], a[2], b[0], b[1], b[2]


def max_rel_err(y, ref):
    """max |y - ref| over the whole output / max |ref| (the north star's measure)."""
    y = y.to(torch.float64)
    ref = ref.to(torch.float64)
    return float((y - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def token_rel_err(y, ref):
    """The same measure per token (row), worst token: a token whose output is
    small next to the batch maximum is held to its own scale."""
    y = y.to(torch.float64).reshape(ref.shape[0], -1)
    ref = ref.to(torch.float64).reshape(ref.shape[0], -1)
    num = (y - ref).abs().amax(dim=1)
    den = ref.abs().amax(dim=1)
    live = den > 0
    if not bool(live.any()):
        return float(num.max())
    return float((num[live] / den[live]).max())


def zipf_routing(T, E, K, seed, alpha=1.2):
    """BASELINE config 5 routing (nanovllm_moe.synthetic.zipf_routing)."""
    from nanovllm_moe.synthetic import zipf_routing as z
    return z(T, E, K, seed, alpha)


def token_sample(T, n, seed, must=()):
    """Sorted sample of n token indices (all when T <= n), plus `must`."""
    if T <= n:
        return list(range(T))
    rng = np.random.default_rng(seed)
    s = set(int(v) for v in rng.choice(T, size=n, replace=False)) | set(int(v) for v in must)
    return sorted(s)
