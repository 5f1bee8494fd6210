"""Seeded synthetic routings for the benchmark configurations.

zipf_routing is BASELINE config 5: expert popularity p_r ~ r^-alpha over a
random permutation of the experts, K distinct experts per token drawn by
Gumbel-top-K over log p, and the softmax of N(0,1) logits as the K weights
(numpy default_rng(seed))."""
import numpy as np
import torch


def zipf_routing(T: int, E: int, K: int, seed: int, alpha: float = 1.2):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    logp = np.empty(E)
    logp[perm] = -alpha * np.log(np.arange(1, E + 1, dtype=np.float64))
    gumbel = -np.log(-np.log(rng.random((T, E))))
    ids = np.argsort(-(logp[None, :] + gumbel), axis=1, kind="stable")[:, :K].astype(np.int32)
    z = rng.standard_normal((T, K))
    w = np.exp(z - z.max(1, keepdims=True))
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return torch.from_numpy(ids), torch.from_numpy(w)
