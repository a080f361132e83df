"""Synthetic caches shaped and distributed as the benchmark configurations of the codec, generated on the device.

These are the inputs bench.py times and the full-size GPU tests check. Every generator draws from a seeded
torch.Generator on the device, so a seed gives the same tensor in every run.

* config 2 (GPT-2-small value cache): Student-t (nu = 5) values, token-major [t][h][d], each head scaled by a
  log-uniform factor in [0.5, 4];
* configs 3 and 5 keys (KIVI): N(0, 1) times per-channel log-normal(sigma = 1) scales, a few outlier channels per
  head at 20x, plus a constant per-head bias vector N(0, 3^2) (a biased key projection);
* config 4 keys (Qwen2.5-1.5B): N(0, 1) plus a per-head bias N(0, 5^2) plus 2 outlier channels per head at 30x;
* config 5 values (Llama-3-8B long context): Student-t (nu = 5), 32 layers x 8 KV heads x 131072 tokens x 128.
"""
from __future__ import annotations

import math

CONFIG5 = dict(layers=32, heads=8, tokens=131072, dim=128)


def student_t(torch, shape, nu: float, gen, device):
    """Student-t(nu) = N(0,1) / sqrt(chi2(nu) / nu). torch's Gamma sampler takes no generator and draws from the
    default generator of the device, which is therefore seeded from gen first."""
    z = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    seed = int(torch.randint(0, 2 ** 62, (1,), generator=gen, device=device).item())
    torch.cuda.manual_seed(seed)
    g = torch.distributions.Gamma(torch.tensor(nu / 2.0, device=device), torch.tensor(0.5, device=device))
    chi2 = g.sample(shape)
    z.div_(torch.sqrt_(chi2.div_(nu)))
    return z


def gpt2_values(torch, gen, device, tokens: int = 32768, heads: int = 12, d: int = 64):
    """Config 2: Student-t (nu = 5) values [t][h][d], scaled per head by log-uniform factors in [0.5, 4]."""
    x = student_t(torch, (tokens, heads, d), 5.0, gen, device)
    f = torch.exp(torch.empty(heads, device=device).uniform_(math.log(0.5), math.log(4.0), generator=gen))
    return (x * f.view(1, heads, 1)).contiguous()


def biased_keys(torch, gen, device, heads: int, tokens: int, d: int, scale_sigma: float = 1.0, outliers: int = 4,
                outlier_x: float = 20.0, bias_sd: float = 3.0, first_head: int = 0):
    """Keys [h][t][d]: N(0,1) * per-channel log-normal(scale_sigma) scales with `outliers` channels per head
    multiplied by outlier_x, plus a per-head bias N(0, bias_sd^2) per channel. The outlier channels of head h are
    drawn from a CPU generator seeded with 1000 + first_head + h, so every head of a multi-layer cache (numbered
    from first_head) has its own."""
    x = torch.randn((heads, tokens, d), generator=gen, device=device)
    s = torch.exp(torch.randn((heads, 1, d), generator=gen, device=device) * scale_sigma)
    for h in range(heads):
        idx = torch.randperm(d, generator=torch.Generator().manual_seed(1000 + first_head + h))[:outliers].to(device)
        s[h, 0, idx] *= outlier_x
    bias = torch.randn((heads, 1, d), generator=gen, device=device) * bias_sd
    return x.mul_(s).add_(bias)


def qwen_keys(torch, gen, device, heads: int, tokens: int, d: int = 128, first_head: int = 0):
    """Config 4 keys: N(0,1) + per-head bias N(0, 5^2) + 2 outlier channels per head at 30x."""
    return biased_keys(torch, gen, device, heads, tokens, d, scale_sigma=0.0, outliers=2, outlier_x=30.0,
                       bias_sd=5.0, first_head=first_head)


def config5_values(torch, gen, device, layers: int = 32, heads: int = 8, tokens: int = 131072, d: int = 128):
    """Config 5 value cache as one [layers][tokens][heads][d] fp32 tensor (token-major per layer, so a token's
    `heads` vectors of a layer are contiguous and an append is one call), Student-t (nu = 5), generated one
    layer at a time."""
    per = tokens * heads
    x = torch.empty((layers * per, d), dtype=torch.float32, device=device)
    for layer in range(layers):
        x[layer * per:(layer + 1) * per] = student_t(torch, (per, d), 5.0, gen, device)
    return x


def config5_keys(torch, gen, device, layers: int = 32, heads: int = 8, tokens: int = 131072, d: int = 128):
    """Config 5 key cache as one [layers][heads][tokens][d] fp32 tensor (head-major, as per-head KIVI groups need),
    with the config-3 distribution drawn per (layer, head): each has its own scales, outlier channels and bias."""
    per = heads * tokens
    x = torch.empty((layers * per, d), dtype=torch.float32, device=device)
    for layer in range(layers):
        x[layer * per:(layer + 1) * per] = biased_keys(torch, gen, device, heads, tokens, d,
                                                       first_head=layer * heads).reshape(per, d)
    return x
