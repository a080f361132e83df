"""The kernels at BASELINE sizes (one GPU's share), checked through size-independent properties.

At full size the oracle cannot check every vector in seconds, so each case checks:
* a sample of rows (the first and last 64, plus 1024 at random) against the oracle: per-vector codes to the
  counted near-boundary band and scales to one float32 ulp, KIVI codes and fp16 ranges bit-exact, and the
  decode of the kernel's own codes within 1e-5 relative L2 (per-vector) or bit-exact (KIVI);
* that encoding a slice through byte offsets into the whole cache gives the same bytes as the whole call;
* the decode/encode error statistics (Theorem 1 band for TurboQuant on Gaussian rows).
Inputs are generated on the device with torch's seeded generator, with the configs' distributions (config 4: a
per-head bias and outlier channels; KIVI keys: per-head scales, outliers and bias). Sizes follow the BASELINE
configs: config 2 (32768 x 12 x 64, TurboQuant b = 2/3/4), config 3 (8 heads x 32768 x 64 KIVI keys, G = 64,
b = 4), config 4 (917,504 x 128, TurboQuant and PolarQuant b = 4), config 5 at one GPU's share under 8-way tensor
parallelism (32 layers x 131072 x 128: V TurboQuant b = 3, K KIVI b = 4), and one call of more than 2^32 floats.
Config 5 at its full single-GPU size is in test_gpu_config5.py.
"""
import math

import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import check_codes, check_scales, max_rel_diff, REL_L2_BAR

pytestmark = pytest.mark.gpu


def _gen(n, d, seed, dev, kind):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    if kind == "gauss":
        return torch.randn(n, d, generator=g, device=dev)
    if kind == "t5":       # Student-t nu = 5 times a per-row log-uniform factor in [0.5, 4]
        from pitch_amd import workloads as W
        x = W.student_t(torch, (n, d), 5.0, g, dev)
        f = torch.exp(torch.empty(n, 1, device=dev).uniform_(math.log(0.5), math.log(4), generator=g))
        return x.mul_(f)
    if kind == "keys":     # per-channel scales, a few outlier channels and a per-channel bias
        z = torch.randn(n, d, generator=g, device=dev)
        s = torch.exp(torch.randn(d, generator=g, device=dev))
        s[:4] *= 20
        return z * s + 3 * torch.randn(d, generator=g, device=dev)
    if kind == "qwen":     # config 4: N(0,1) + per-head bias N(0, 5^2) + 2 outlier channels per head at 30x
        from pitch_amd import workloads as W
        heads = 56         # 28 layers x 2 KV heads, head-major rows
        assert n % heads == 0
        return W.qwen_keys(torch, g, dev, heads, n // heads, d).reshape(n, d)
    raise ValueError(kind)


def _sample(n, seed):
    rng = np.random.default_rng(seed)
    idx = np.concatenate([np.arange(min(64, n)), np.arange(max(0, n - 64), n), rng.integers(0, n, 1024)])
    return np.unique(idx)


def per_vector_full(q, method, n, d, bits, seed, kind="gauss", theorem1=False):
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"full-size {method} n={n} d={d} b={bits}", flush=True)
    cfg = P.QuantConfig(method, d, bits)
    x = _gen(n, d, seed, dev, kind).contiguous()
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    out = torch.empty(n, d, dtype=torch.float32, device=dev)
    q.enqueueEncode(x, codes, scales, n, cfg)
    q.enqueueDecode(codes, scales, out, n, cfg)
    torch.cuda.synchronize()
    idx = _sample(n, seed)
    it = torch.from_numpy(idx).to(dev)
    X = x[it].cpu().numpy()
    C = codes.view(n, cfg.codeStride)[it].cpu().numpy().tobytes()
    S = scales[it].cpu().numpy()
    ref_codes, ref_scales = O.ENCODERS[method](X.astype(np.float64), bits)
    check_codes(method, X, bits, P.DEFAULT_SEED, C, O.pack_codes(ref_codes, bits), f"{method} n={n}")
    check_scales(S, np.asarray(ref_scales, np.float32), "scales")
    ours = O.unpack_codes(C, len(idx), d, bits)
    recon = O.DECODERS[method](ours, S.astype(np.float64), bits)
    assert max_rel_diff(out[it].cpu().numpy(), recon, d) < REL_L2_BAR
    # a slice encoded through byte offsets equals the same bytes of the whole call
    lo, m = n // 3, min(n // 3, 100003)
    c2 = torch.zeros(m * cfg.codeStride, dtype=torch.uint8, device=dev)
    s2 = torch.zeros(m, dtype=torch.float32, device=dev)
    q.enqueueEncode(x, c2, s2, m, cfg, inputOffset=lo * d * 4)
    torch.cuda.synchronize()
    assert torch.equal(c2, codes[lo * cfg.codeStride:(lo + m) * cfg.codeStride])
    assert torch.equal(s2, scales[lo:lo + m])
    if theorem1:
        num = (x - out).double().square().sum(1)
        den = x.double().square().sum(1)
        e = float((num / den).mean())
        assert 4.0 ** -bits <= e <= math.sqrt(3) * math.pi / 2 * 4.0 ** -bits
    del x, codes, scales, out, c2, s2
    torch.cuda.empty_cache()


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_config2_gpt2_v_cache(q, bits):
    per_vector_full(q, "turboQuant", 32768 * 12, 64, bits, 2000 + bits, "t5")


@pytest.mark.parametrize("method", ["turboQuant", "polarQuant"])
def test_config4_qwen_d128(q, method):
    """Config 4 on its own key distribution (a per-head bias and two outlier channels per head)."""
    per_vector_full(q, method, 28 * 2 * 16384, 128, 4, 4000, "qwen")


def test_config4_shape_gaussian_theorem1(q):
    """Config 4's shape on N(0,1) rows, where TurboQuant's mean error is inside the Theorem-1 band."""
    per_vector_full(q, "turboQuant", 28 * 2 * 16384, 128, 4, 4001, "gauss", theorem1=True)


def test_config5_v_share(q):
    per_vector_full(q, "turboQuant", 32 * 131072, 128, 3, 5000, "t5")


@pytest.mark.parametrize("method,d,bits", [("polarQuant", 128, 4), ("turboQuant", 64, 4), ("polarQuant", 64, 3),
                                           ("turboQuant", 64, 3)])
def test_long_calls_oversubscribed_grid(q, method, d, bits):
    """The staged encoder runs calls of at least 56 resident rounds as one launch of about 8 blocks per workgroup
    (encode_grid): 3 * 2^20 vectors are 49,152 blocks of 64, 64 rounds of 768 resident workgroups on a 256-CU
    device. Sampled rows match the oracle, and the slice per_vector_full encodes through byte offsets (100,003
    vectors, a persistent grid) gives the same bytes as the long call."""
    per_vector_full(q, method, 3 << 20, d, bits, 7000 + d + bits, "t5")


def test_more_than_2_32_floats_in_one_call(q):
    """count * dim > 2^32 (a documented extension: the reference caps a call below 2^32 elements)."""
    per_vector_full(q, "turboQuant", (1 << 22) + 100, 1024, 4, 6000, "gauss")


def channel_full(q, heads, tokens, d, bits, G, seed, one_call=False):
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"full-size KIVI heads={heads} tokens={tokens} d={d} b={bits} G={G}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(tokens)
    # the config-3 distribution drawn per head: each head has its own scales, outlier channels and bias
    from pitch_amd import workloads as W
    gk = torch.Generator(device=dev).manual_seed(seed)
    x = W.biased_keys(torch, gk, dev, heads, tokens, d, first_head=seed).reshape(heads * tokens, d).contiguous()
    codes = torch.empty(heads * tokens * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.empty(heads * groups * cfg.rangeStride // 2, dtype=torch.float16, device=dev)
    out = torch.empty(heads * tokens, d, dtype=torch.float32, device=dev)
    if one_call:                     # all heads in one call: groups never cross a head (tokens % G == 0)
        assert tokens % G == 0
        q.enqueuePerChannelEncode(x, codes, ranges, heads * tokens, cfg)
        q.enqueuePerChannelDecode(codes, ranges, out, heads * tokens, cfg)
    for h in range(0 if one_call else heads):   # one call per head, at its offsets in the whole cache
        q.enqueuePerChannelEncode(x, codes, ranges, tokens, cfg, inputOffset=h * tokens * d * 4,
                                  codesOffset=h * tokens * cfg.codeStride, rangesOffset=h * groups * cfg.rangeStride)
        q.enqueuePerChannelDecode(codes, ranges, out, tokens, cfg, codesOffset=h * tokens * cfg.codeStride,
                                  rangesOffset=h * groups * cfg.rangeStride, outputOffset=h * tokens * d * 4)
    torch.cuda.synchronize()
    rng = np.random.default_rng(seed)
    picks = [(0, 0), (heads - 1, groups - 1)] + [(int(rng.integers(heads)), int(rng.integers(groups)))
                                                   for _ in range(14)]
    for h, g in picks:
        t0 = h * tokens + g * G
        m = min(G, tokens - g * G)
        X = x[t0:t0 + m].cpu().numpy()
        ref_codes, ref_ranges = O.channel_encode(X, bits, G)
        got_c = codes[t0 * cfg.codeStride:(t0 + m) * cfg.codeStride].cpu().numpy().tobytes()
        assert got_c == O.pack_codes(ref_codes, bits), (h, g)
        r0 = (h * groups + g) * 2 * d
        got_r = ranges[r0:r0 + 2 * d].cpu().numpy().view(np.uint16)
        assert np.array_equal(got_r, ref_ranges.view(np.uint16).reshape(-1)), (h, g)
        ref = O.channel_decode(ref_codes, ref_ranges, bits, G)
        assert np.array_equal(out[t0:t0 + m].cpu().numpy().view(np.uint32), ref.view(np.uint32)), (h, g)
    del x, codes, ranges, out
    torch.cuda.empty_cache()


def test_config3_kivi_keys(q):
    channel_full(q, 8, 32768, 64, 4, 64, 3000)


def test_config5_k_share(q):
    channel_full(q, 32, 131072, 128, 4, 64, 5001)


def test_kivi_long_call_one_launch_matches_per_head_calls(q):
    """Float32 KIVI encodes of at least 16 resident rounds run one launch of one item per wave: 32 heads x 131,072
    tokens at d = 128 are 131,072 (group, 64-channel slab) items, 32,768 workgroups, 32 rounds of 1,024 on a
    256-CU device. The long call's codes and ranges equal, byte for byte, those of one call per head (131,072 tokens
    each, a persistent grid), and sampled groups of a long call match the oracle (channel_full, one_call)."""
    import torch
    import pitch_amd as P
    from pitch_amd import workloads as W
    heads, tokens, d, bits, G = 32, 131072, 128, 4, 64
    dev = q.device
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(tokens)
    gk = torch.Generator(device=dev).manual_seed(5201)
    x = W.biased_keys(torch, gk, dev, heads, tokens, d).reshape(heads * tokens, d).contiguous()
    c1 = torch.empty(heads * tokens * cfg.codeStride, dtype=torch.uint8, device=dev)
    r1 = torch.empty(heads * groups * cfg.rangeStride // 2, dtype=torch.float16, device=dev)
    c2 = torch.zeros_like(c1)
    r2 = torch.zeros_like(r1)
    q.enqueuePerChannelEncode(x, c1, r1, heads * tokens, cfg)
    for h in range(heads):
        q.enqueuePerChannelEncode(x, c2, r2, tokens, cfg, inputOffset=h * tokens * d * 4,
                                  codesOffset=h * tokens * cfg.codeStride, rangesOffset=h * groups * cfg.rangeStride)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    assert torch.equal(r1.view(torch.int16), r2.view(torch.int16))
    del x, c1, r1, c2, r2
    torch.cuda.empty_cache()
    channel_full(q, heads, tokens, d, bits, G, 5202, one_call=True)


@pytest.mark.parametrize("d,bits,n", [(128, 4, (1 << 23) + 37), (64, 3, (1 << 24) + 100)])
def test_kivi_long_decode_one_launch_matches_slices(q, d, bits, n):
    """Float32 KIVI decodes of at least 8 resident rounds (about 65,536 (group, 64-channel) items or more) run one
    launch of one item per wave with a capped residency. The long call's output equals, byte for byte, the decode of
    the same codes in slices of 2^18 tokens (2 rounds or fewer: one launch at full residency), the partial last group
    included. Codes are random bytes and ranges random finite fp16 pairs, so every code value occurs."""
    import torch
    import pitch_amd as P
    G = 64
    dev = q.device
    print(f"long KIVI decode d={d} b={bits} tokens={n}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(n)
    g = torch.Generator(device=dev).manual_seed(5300 + d + bits)
    codes = torch.randint(0, 256, (n * cfg.codeStride,), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    lo = torch.randn(groups, 1, d, generator=g, device=dev) * 3
    hi = lo + torch.rand(groups, 1, d, generator=g, device=dev) * 4
    ranges = torch.cat([lo, hi], 1).half().reshape(-1)
    del lo, hi
    out = torch.full((n, d), float("nan"), dtype=torch.float32, device=dev)
    ref = torch.full((n, d), float("nan"), dtype=torch.float32, device=dev)
    q.enqueuePerChannelDecode(codes, ranges, out, n, cfg)
    per = 1 << 18
    for t0 in range(0, n, per):
        m = min(per, n - t0)
        q.enqueuePerChannelDecode(codes, ranges, ref, m, cfg, codesOffset=t0 * cfg.codeStride,
                                  rangesOffset=(t0 // G) * cfg.rangeStride, outputOffset=t0 * d * 4)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32))


@pytest.mark.parametrize("bits", [4, 3])
def test_kivi_long_encode_one_launch_partial_group(q, bits):
    """A float32 KIVI encode of 16+ resident rounds (one launch at a capped residency, 64-channel slabs) ending in a
    partial group: 2^22 + 37 tokens at d = 128 are 131,074 (group, 64-channel) items. Codes and ranges equal, byte
    for byte, those of the same keys encoded in slices of 2^18 tokens (32-channel slabs, one launch at full
    residency), and the last (37-token) group and the first one match the oracle bit for bit."""
    kivi_encode_vs_slices(q, 128, bits, (1 << 22) + 37, 1 << 18, 5400 + bits)


@pytest.mark.parametrize("d,bits", [(64, 4), (128, 3), (64, 2)])
def test_kivi_mid_encode_one_launch_partial_group(q, d, bits):
    """A float32 KIVI encode of 4-16 resident rounds of 32-channel slabs (one launch at the encoder's full
    residency): 2^19 + 37 tokens. Codes and ranges equal, byte for byte, those of slices of 2^17 tokens (the
    balanced persistent grid), and the first and last (37-token) groups match the oracle bit for bit."""
    kivi_encode_vs_slices(q, d, bits, (1 << 19) + 37, 1 << 17, 5500 + d + bits)


def kivi_encode_vs_slices(q, d, bits, n, per, seed):
    import torch
    import pitch_amd as P
    from pitch_amd import workloads as W
    G = 64
    dev = q.device
    print(f"KIVI encode d={d} b={bits} tokens={n} against slices of {per}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(n)
    gk = torch.Generator(device=dev).manual_seed(seed)
    x = W.biased_keys(torch, gk, dev, 1, n, d).reshape(n, d).contiguous()
    c1 = torch.zeros(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    r1 = torch.full((groups * 2 * d,), float("nan"), dtype=torch.float16, device=dev)
    c2 = torch.zeros_like(c1)
    r2 = torch.full_like(r1, float("nan"))
    q.enqueuePerChannelEncode(x, c1, r1, n, cfg)
    for t0 in range(0, n, per):
        m = min(per, n - t0)
        q.enqueuePerChannelEncode(x, c2, r2, m, cfg, inputOffset=t0 * d * 4, codesOffset=t0 * cfg.codeStride,
                                  rangesOffset=(t0 // G) * cfg.rangeStride)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    assert torch.equal(r1.view(torch.int16), r2.view(torch.int16))
    for g in (0, groups - 1):
        t0 = g * G
        m = min(G, n - t0)
        ref_codes, ref_ranges = O.channel_encode(x[t0:t0 + m].cpu().numpy(), bits, G)
        got = c1[t0 * cfg.codeStride:(t0 + m) * cfg.codeStride].cpu().numpy().tobytes()
        assert got == O.pack_codes(ref_codes, bits), g
        rr = r1.view(groups, 2, d)[g].cpu().numpy()
        assert np.array_equal(rr.view(np.uint16), np.asarray(ref_ranges, np.float16).reshape(2, d).view(np.uint16)), g


@pytest.mark.parametrize("bits", [2, 3, 8])
def test_kivi_64_channel_slabs_bit_widths(q, bits):
    """One call of 2^21 + 192 tokens at d = 64: 32,771 (group, 64-channel) items, so the encoder takes its
    64-channel-slab variant, here at the bit widths whose lane fields are packed directly (2, 8) and one that
    goes through byte staging (3)."""
    channel_full(q, 1, (1 << 21) + 192, 64, bits, 64, 5100 + bits, one_call=True)


def test_config5_k_share_one_call(q):
    """16 heads x 131072 tokens in one call: 65,536 (group, 64-channel) items, so the encoder takes its
    64-channel-slab variant (fewer items take the 32-channel one, covered above)."""
    channel_full(q, 16, 131072, 128, 4, 64, 5002, one_call=True)


@pytest.mark.parametrize("d,bits,G", [(128, 4, 64), (64, 3, 64), (96, 2, 32), (128, 8, 128)])
def test_kivi_long_call_partial_last_group(q, d, bits, G):
    """One call long enough to be issued as several launches (the wave kernels split calls of more than two rounds),
    ending in a partial group: codes, ranges and decode bit-exact against the oracle at the first, last and
    launch-boundary-straddling groups and at random ones."""
    import torch
    import pitch_amd as P
    dev = q.device
    n = (1 << 21) + 37 if d <= 96 else (1 << 20) + 37
    print(f"long KIVI call d={d} b={bits} G={G} tokens={n}", flush=True)
    cfg = P.ChannelQuantConfig(d, bits, G)
    groups = cfg.groupCount(n)
    x = _gen(n, d, 7000 + d + bits, dev, "keys").contiguous()
    codes = torch.zeros(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.full((groups * 2 * d,), float("nan"), dtype=torch.float16, device=dev)
    out = torch.full((n, d), float("nan"), dtype=torch.float32, device=dev)
    q.enqueuePerChannelEncode(x, codes, ranges, n, cfg)
    q.enqueuePerChannelDecode(codes, ranges, out, n, cfg)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all()) and bool(torch.isfinite(ranges).all())
    # every group's fp16 range: the float32 min / max rounded to nearest even (pitch_reference.py:150-153), so a
    # group skipped or written to the wrong place by any launch shows up
    full = (n // G) * G
    xg = x[:full].view(-1, G, d)
    r = ranges.view(groups, 2, d)
    assert torch.equal(r[:n // G, 0], xg.amin(1).half()) and torch.equal(r[:n // G, 1], xg.amax(1).half())
    if n % G:
        assert torch.equal(r[-1, 0], x[full:].amin(0).half()) and torch.equal(r[-1, 1], x[full:].amax(0).half())
    # every element within half a step (plus the fp16 rounding of the range ends) of its input
    rf = r.float()
    step = ((rf[:, 1] - rf[:, 0]) / (2 ** bits - 1)).clamp_min(0)
    tol = (0.5 * step * (1 + 1e-5) + 4.9e-4 * torch.maximum(rf[:, 0].abs(), rf[:, 1].abs()) + 6e-8)
    tol = tol.repeat_interleave(G, 0)[:n]
    assert not bool(((x - out).abs() > tol).any())
    del xg, r, rf, step, tol
    rng = np.random.default_rng(d + bits)
    picks = sorted({0, 1, groups - 2, groups - 1} | {int(g) for g in rng.integers(0, groups, 40)}
                   | {k * 256 + o for k in range(1, groups // 256) for o in (-1, 0)})
    for g in picks:
        t0 = g * G
        m = min(G, n - t0)
        X = x[t0:t0 + m].cpu().numpy()
        ref_codes, ref_ranges = O.channel_encode(X, bits, G)
        got_c = codes[t0 * cfg.codeStride:(t0 + m) * cfg.codeStride].cpu().numpy().tobytes()
        assert got_c == O.pack_codes(ref_codes, bits), g
        got_r = ranges[g * 2 * d:(g + 1) * 2 * d].cpu().numpy().view(np.uint16)
        assert np.array_equal(got_r, ref_ranges.view(np.uint16).reshape(-1)), g
        ref = O.channel_decode(ref_codes, ref_ranges, bits, G)
        assert np.array_equal(out[t0:t0 + m].cpu().numpy().view(np.uint32), ref.view(np.uint32)), g
    del x, codes, ranges, out
    torch.cuda.empty_cache()
