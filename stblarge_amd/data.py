"""Seeded synthetic inputs for the path's configurations (no checkpoints, no datasets).

Every tensor is a function of an integer seed. Weights are N(0, 0.02) fp32, activations N(0, 1)
rounded to bf16, router logits follow the Zipf(1.1) Gumbel-top-k construction. Generation runs with
torch's Philox generator on the device the tensor is made on; the CPU variant (device="cpu") is what
the parity tests feed to both the oracle and the GPU.
"""

import math

import torch

DIM, INTER = 7168, 2048          # expert shapes: gate/up [INTER x DIM], down [DIM x INTER]
N_EXPERTS, TOPK, CACHE_SLOTS = 256, 8, 64


def generator(seed, device):
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def normal(shape, std, seed, device="cpu"):
    g = generator(seed, device)
    return torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std


def weight(rows, k, seed, device="cpu"):
    """W ~ N(0, 0.02) fp32 [rows, k]."""
    return normal((rows, k), 0.02, seed, device)


def activation(m, k, seed, device="cpu"):
    """x ~ N(0, 1) rounded to bf16, [m, k]."""
    return normal((m, k), 1.0, seed, device).to(torch.bfloat16)


def zipf_logits(tokens, n_experts, seed, alpha=1.1, device="cpu"):
    """Router logits whose sigmoid top-k is a Zipf(alpha) sample without replacement.

    l_e = log p_{pi(e)} + Gumbel_e with p_r ~ r^-alpha over ranks r = 1..E and pi a seeded permutation
    of the experts; the k largest l_e (and so the k largest sigmoid(l_e)) are a weighted sample
    without replacement with weights p (the Gumbel-top-k construction)."""
    g = generator(seed, "cpu")
    ranks = torch.arange(1, n_experts + 1, dtype=torch.float64)
    logp = -alpha * torch.log(ranks)
    logp = logp - torch.logsumexp(logp, 0)
    perm = torch.randperm(n_experts, generator=g)
    u = torch.rand((tokens, n_experts), generator=g, dtype=torch.float64).clamp_min(1e-300)
    gumbel = -torch.log(-torch.log(u))
    logits = logp[perm].unsqueeze(0) + gumbel
    return logits.to(torch.float32).to(device)


def algorithmic_bytes_fp4(n, k, m=1):
    """Codes + E8M0 scales + bf16 x + bf16 y: each byte counted once."""
    return n * k // 2 + n * k // 32 + 2 * k * m + 2 * n * m


def algorithmic_bytes_fp8(n, k, m=1):
    """Codes + fp32 128x128 block scales + bf16 x + bf16 y."""
    return n * k + 4 * math.ceil(n / 128) * math.ceil(k / 128) + 2 * k * m + 2 * n * m
