"""Writes the golden fixtures in this directory.

The reference holds no golden vectors for this path (its tests assert shapes
and dtypes only, Int8-gemm/test/fused_moe_cpu.py:164-165), and its CPU code is
ARM-only, so the expected values here come from a numpy restatement written
independently of the C oracle and of the HIP kernels:

  golden_q8_0.npz     Q8_0 block quantization (Int8-gemm/gemm_kernels.cpp:
                      25-58): amax, d = amax/127 (fp32), id = 1/d (0 if d=0),
                      q = saturate(round-half-even(x*id)).  Inputs are
                      bf16-exact; special blocks: zeros, +-amax, exact ties,
                      tiny, huge, single spike.
  golden_route.npz    preprocess_moe_routing (Int8-gemm/moe_common.cpp:
                      146-216) as a stable argsort by expert over (t, k)
                      order, with invalid ids dropped.
  golden_q4_dots.npz  per-32-block int32 dots of Q8_0 activations against
                      Q4_0 wire words (element k in word k/8, nibble k%8,
                      value nibble-8; Int8-gemm/gemm_kernels.cpp:542).
  golden_w4a16.npz    a small W4A16 layer (AWQ wire tensors, group 128) and
                      its output from a float64 dense formula:
                      y[t] = sum_k w[t,k] W2[e] (up * silu(gate)), gate/up
                      = halves of W13[e] x[t], W = (q - z) * s.

Run from the repository root:  python tests/golden/make_golden.py
Generator: numpy default_rng, seeds listed per fixture.
"""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
AWQ_SLOT = [0, 4, 1, 5, 2, 6, 3, 7]   # column n%8 of a group of 8 -> nibble slot


def bf16_round(x):
    """float32 -> nearest bf16 (ties to even), returned as float32 and bits."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return (r.astype(np.uint32) << 16).view(np.float32), r


def q8_0_blocks(x):
    x = np.asarray(x, np.float32)
    amax = np.abs(x).max(axis=-1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    idv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    prod = (x * idv[..., None]).astype(np.float32)
    q = np.clip(np.rint(prod), -128, 127).astype(np.int8)
    return q, d


def make_q8_0(rng):
    blocks = []
    blocks.append(np.zeros(32, np.float32))                                  # zero block
    b = rng.standard_normal(32).astype(np.float32); b[5] = 3.0; b[9] = -3.0
    blocks.append(b)                                                         # +-amax
    blocks.append(np.arange(-16, 16, dtype=np.float32) * 0.5)                # multiples of 0.5
    ties = np.array([127.0] + [s * (h + 0.5) for h in range(8) for s in (1, -1)] + [0.0] * 15, np.float32)
    blocks.append(ties)                                                      # d = 1: exact .5 ties -> even
    blocks.append(np.full(32, 1e-30, np.float32))                            # tiny
    blocks.append((rng.standard_normal(32) * 1e30).astype(np.float32))       # huge
    spike = np.zeros(32, np.float32); spike[31] = -2.5
    blocks.append(spike)
    for _ in range(57):
        blocks.append((rng.standard_normal(32) * rng.choice([0.01, 1.0, 30.0])).astype(np.float32))
    x = np.stack(blocks)
    xb, bits = bf16_round(x)
    q, d = q8_0_blocks(xb)
    np.savez(os.path.join(HERE, "golden_q8_0.npz"), x_bf16_bits=bits, x=xb, qs=q, d=d, seed=np.int64(1))


def make_route(rng):
    T, K, E = 37, 8, 16
    ids = rng.integers(0, E, size=(T, K)).astype(np.int32)
    ids[3, 2] = -1
    ids[7, :] = E + 3          # token with no valid id
    ids[11, 4] = ids[11, 5]    # repeated expert inside a token
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    counts = np.bincount(flat[valid], minlength=E).astype(np.int32)
    starts = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    order = np.argsort(np.where(valid, flat, E), kind="stable")[: int(valid.sum())]
    token_map = np.stack([order // K, order % K], axis=1).astype(np.int32)
    scatter = np.full(T * K, -1, np.int32)
    scatter[order] = np.arange(order.size, dtype=np.int32)
    np.savez(os.path.join(HERE, "golden_route.npz"), ids=ids, E=np.int64(E), counts=counts,
             starts=starts, token_map=token_map, scatter=scatter.reshape(T, K), seed=np.int64(2))


def make_q4_dots(rng):
    M, N, K = 4, 64, 128
    vals = rng.integers(-8, 8, size=(N, K))
    nib = (vals + 8).astype(np.uint64).reshape(N, K // 8, 8)
    words = (nib << (4 * np.arange(8, dtype=np.uint64))).sum(axis=-1).astype(np.uint32).view(np.int32)
    a = rng.integers(-128, 128, size=(M, K)).astype(np.int8)
    isum = np.einsum("mbi,nbi->mnb", a.astype(np.int64).reshape(M, K // 32, 32),
                     vals.astype(np.int64).reshape(N, K // 32, 32)).astype(np.int32)
    np.savez(os.path.join(HERE, "golden_q4_dots.npz"), w_words=words, a_qs=a, isum=isum,
             seed=np.int64(3))


def awq_pack(q):
    """[..., N] nibbles -> int32 [..., N/8] in the AWQ order."""
    *lead, n = q.shape
    q = q.astype(np.uint64).reshape(*lead, n // 8, 8)
    out = np.zeros((*lead, n // 8), np.uint64)
    for col, slot in enumerate(AWQ_SLOT):
        out |= q[..., col] << np.uint64(4 * slot)
    return out.astype(np.uint32).view(np.int32)


def make_w4a16(rng):
    E, H, I, T, K, g = 2, 512, 128, 3, 2, 128

    def layer(N, Kd):
        q = rng.integers(0, 16, size=(E, Kd, N))
        z = rng.integers(0, 16, size=(E, Kd // g, N))
        s, s_bits = bf16_round((rng.random((E, Kd // g, N)) * 0.004 + 0.001).astype(np.float32))
        w = (q - np.repeat(z, g, axis=1)).astype(np.float64) * np.repeat(s, g, axis=1).astype(np.float64)
        return awq_pack(q), awq_pack(z), s_bits, np.transpose(w, (0, 2, 1))   # W [E, N, K]

    w13_q, w13_z, w13_s, W13 = layer(2 * I, H)
    w2_q, w2_z, w2_s, W2 = layer(H, I)
    x, x_bits = bf16_round(rng.standard_normal((T, H)).astype(np.float32))
    logits = rng.standard_normal((T, E))
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :K].astype(np.int32)
    top = np.take_along_axis(logits, ids, axis=1)
    tw = (np.exp(top - top.max(1, keepdims=True)) / np.exp(top - top.max(1, keepdims=True)).sum(1, keepdims=True)).astype(np.float32)
    y = np.zeros((T, H))
    for t in range(T):
        for k in range(K):
            e = ids[t, k]
            gu = W13[e] @ x[t].astype(np.float64)
            act = gu[I:] * (gu[:I] / (1.0 + np.exp(-gu[:I])))
            y[t] += float(tw[t, k]) * (W2[e] @ act)
    np.savez(os.path.join(HERE, "golden_w4a16.npz"), E=np.int64(E), H=np.int64(H), I=np.int64(I),
             group=np.int64(g), w13_q=w13_q, w13_z=w13_z, w13_s_bf16=w13_s, w2_q=w2_q, w2_z=w2_z,
             w2_s_bf16=w2_s, x_bf16_bits=x_bits, topk_ids=ids, topk_w=tw, y=y.astype(np.float32),
             seed=np.int64(4))


if __name__ == "__main__":
    make_q8_0(np.random.default_rng(1))
    make_route(np.random.default_rng(2))
    make_q4_dots(np.random.default_rng(3))
    make_w4a16(np.random.default_rng(4))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
