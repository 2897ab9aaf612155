"""Seeded synthetic Q4_K weights and activations for the benchmark configs.

The configs specify (per super-block): fp16 d and dmin drawn from
|N(0, 0.02)|, 12 uniform random bytes of packed 6-bit scales/mins (every
6-bit field uniform on [0, 63]) and 128 uniform random bytes of nibbles.
`q4k_random_np` draws them on the host with numpy's PCG64; `q4k_random_dev`
draws them on the GPU with a seeded torch generator (used for the multi-GB
expert stacks).  Both return [n_blocks, 144] uint8.
"""
import numpy as np


def q4k_random_np(rng, n_blocks):
    b = rng.integers(0, 256, size=(n_blocks, 144), dtype=np.uint8)
    dd = np.abs(rng.normal(0.0, 0.02, size=(n_blocks, 2))).astype(np.float16)
    b[:, 0:4] = dd.view(np.uint8).reshape(n_blocks, 4)
    return b


def q4k_random_dev(n_blocks, gen, device="cuda", out=None):
    import torch
    if out is None:
        out = torch.empty((n_blocks, 144), dtype=torch.uint8, device=device)
    step = 1 << 22
    for s in range(0, n_blocks, step):
        e = min(n_blocks, s + step)
        v = out[s:e]
        v.copy_(torch.randint(0, 256, (e - s, 144), dtype=torch.uint8, device=device,
                              generator=gen))
        dd = (torch.randn((e - s, 2), device=device, generator=gen) * 0.02).abs().half()
        v[:, 0:4] = dd.view(torch.uint8).reshape(e - s, 4)
    return out


def q6k_random_np(rng, n_blocks):
    """Q6_K blocks: uniform ql/qh bytes, int8 scales uniform in [-128, 127],
    d = fp16(|N(0, 0.002)|)."""
    b = rng.integers(0, 256, size=(n_blocks, 210), dtype=np.uint8)
    d = np.abs(rng.normal(0.0, 0.002, size=(n_blocks, 1))).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(n_blocks, 2)
    return b


def q6k_random_dev(n_blocks, gen, device="cuda", out=None):
    import torch
    if out is None:
        out = torch.empty((n_blocks, 210), dtype=torch.uint8, device=device)
    step = 1 << 22
    for s in range(0, n_blocks, step):
        e = min(n_blocks, s + step)
        v = out[s:e]
        v.copy_(torch.randint(0, 256, (e - s, 210), dtype=torch.uint8, device=device,
                              generator=gen))
        d = (torch.randn((e - s, 1), device=device, generator=gen) * 0.002).abs().half()
        v[:, 208:210] = d.view(torch.uint8).reshape(e - s, 2)
    return out


def zipf_routes(rng, n_layers, n_expert, k, s=1.1):
    """Per layer, k distinct experts sampled without replacement from a
    Zipf(s) popularity over a seeded permutation of the experts (Gumbel
    top-k on log-popularity)."""
    ranks = np.arange(1, n_expert + 1, dtype=np.float64)
    logp = -s * np.log(ranks)
    out = np.zeros((n_layers, k), np.int32)
    for L in range(n_layers):
        perm = rng.permutation(n_expert)
        g = logp + rng.gumbel(size=n_expert)
        top = np.argsort(-g, kind="stable")[:k]
        out[L] = perm[top]
    return out
