"""Config 5 (Llama-3-8B long context) at its full single-GPU size, each cache in ONE call.

V: TurboQuant d = 128, b = 3 over 32 layers x 8 KV heads x 131072 tokens = 33,554,432 vectors (2^32 floats,
17.2 GB), real Student-t (nu = 5) values. K: KIVI d = 128, b = 4, G = 64 over the same 33,554,432 tokens, the
config-3 distribution drawn per (layer, head). One call covers 2^32 floats, beyond the reference's per-call limit
count * dim <= 2^32 - 1 (Sources/PITCH/Core/Codec.swift:30-32, PerChannel.swift:309-316); this build's 64-bit
addressing lifts it.

Checks (the oracle cannot process 33.5M vectors in seconds):
* sampled rows against the oracle: the first and last 64 rows, the rows around every layer boundary, and 1024
  at random. Per-vector codes to the counted near-boundary band, scales to one float32 ulp, and the decode of
  the kernel's own codes within 1e-5 relative L2. KIVI: codes, fp16 ranges and decode bit-exact for the first and
  last group, the groups at every (layer, head) boundary, and 64 at random;
* every row, through size-independent properties: outputs pre-filled with NaN and scales with -1 are all
  overwritten with finite values; every TurboQuant vector decodes within relative L2 0.6 of its input (b = 3:
  typically 0.18; a stale or misplaced code row lands near 1.4); every KIVI element decodes within half a step
  (plus the fp16 rounding of its range ends) of its input, and every group's fp16 range has lo <= hi.
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import check_codes, check_scales, max_rel_diff, REL_L2_BAR

pytestmark = pytest.mark.gpu

L, H, T, D = 32, 8, 131072, 128
N = L * H * T


def _rows(seed):
    rng = np.random.default_rng(seed)
    per = H * T
    idx = [np.arange(64), np.arange(N - 64, N), rng.integers(0, N, 1024)]
    idx += [np.arange(max(0, layer * per - 2), min(N, layer * per + 2)) for layer in range(1, L)]
    return np.unique(np.concatenate(idx))


def test_config5_values_one_call(q):
    import torch
    import pitch_amd as P
    from pitch_amd import workloads as W
    dev = q.device
    print(f"config 5 V: TurboQuant d=128 b=3, {N} vectors in one call: generating", flush=True)
    gen = torch.Generator(device=dev).manual_seed(55)
    x = W.config5_values(torch, gen, dev)
    cfg = P.QuantConfig("turboQuant", D, 3)
    codes = torch.zeros(N * cfg.codeStride, dtype=torch.uint8, device=dev)
    scales = torch.full((N,), -1.0, dtype=torch.float32, device=dev)
    out = torch.full((N, D), float("nan"), dtype=torch.float32, device=dev)
    print("config 5 V: encode + decode", flush=True)
    q.enqueueEncode(x, codes, scales, N, cfg)
    q.enqueueDecode(codes, scales, out, N, cfg)
    torch.cuda.synchronize()
    print("config 5 V: sampled rows vs the oracle", flush=True)
    idx = _rows(5)
    it = torch.from_numpy(idx).to(dev)
    X = x[it].cpu().numpy()
    C = codes.view(N, cfg.codeStride)[it].cpu().numpy().tobytes()
    S = scales[it].cpu().numpy()
    ref_codes, ref_scales = O.turbo_encode(X.astype(np.float64), 3)
    diffs = check_codes("turboQuant", X, 3, P.DEFAULT_SEED, C, O.pack_codes(ref_codes, 3), "config 5 V")
    check_scales(S, np.asarray(ref_scales, np.float32), "config 5 V scales")
    recon = O.turbo_decode(O.unpack_codes(C, len(idx), D, 3), S.astype(np.float64), 3)
    assert max_rel_diff(out[it].cpu().numpy(), recon, D) < REL_L2_BAR
    print(f"config 5 V: {diffs} near-boundary code differences in {len(idx)} rows; every row", flush=True)
    assert bool((scales >= 0).all()) and bool(torch.isfinite(scales).all())
    worst = 0.0
    for layer in range(L):                      # per layer: no 17 GB temporaries
        a, b = layer * H * T, (layer + 1) * H * T
        xs, os_ = x[a:b].double(), out[a:b].double()
        assert bool(torch.isfinite(out[a:b]).all()), f"layer {layer}: unwritten or non-finite output"
        e = ((xs - os_).square().sum(1) / xs.square().sum(1).clamp_min(1e-300)).sqrt()
        worst = max(worst, float(e.max()))
        del xs, os_, e
    print(f"config 5 V: worst per-vector relative L2 error {worst:.3f}", flush=True)
    assert worst < 0.6
    del x, codes, scales, out
    torch.cuda.empty_cache()


def test_config5_keys_one_call(q):
    import torch
    import pitch_amd as P
    from pitch_amd import workloads as W
    dev = q.device
    G, bits = 64, 4
    print(f"config 5 K: KIVI d=128 b=4 G=64, {N} tokens in one call: generating", flush=True)
    gen = torch.Generator(device=dev).manual_seed(56)
    x = W.config5_keys(torch, gen, dev)
    cfg = P.ChannelQuantConfig(D, bits, G)
    groups = cfg.groupCount(N)
    codes = torch.zeros(N * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.full((groups * 2 * D,), float("nan"), dtype=torch.float16, device=dev)
    out = torch.full((N, D), float("nan"), dtype=torch.float32, device=dev)
    print("config 5 K: encode + decode", flush=True)
    q.enqueuePerChannelEncode(x, codes, ranges, N, cfg)
    q.enqueuePerChannelDecode(codes, ranges, out, N, cfg)
    torch.cuda.synchronize()
    print("config 5 K: sampled groups vs the oracle", flush=True)
    rng = np.random.default_rng(57)
    per_head = T // G
    picks = {0, groups - 1} | {int(g) for g in rng.integers(0, groups, 64)}
    picks |= {lh * per_head + o for lh in range(1, L * H) for o in (-1, 0)}
    for g in sorted(picks):
        t0 = g * G
        X = x[t0:t0 + G].cpu().numpy()
        ref_codes, ref_ranges = O.channel_encode(X, bits, G)
        got_c = codes[t0 * cfg.codeStride:(t0 + G) * cfg.codeStride].cpu().numpy().tobytes()
        assert got_c == O.pack_codes(ref_codes, bits), g
        got_r = ranges[g * 2 * D:(g + 1) * 2 * D].cpu().numpy().view(np.uint16)
        assert np.array_equal(got_r, ref_ranges.view(np.uint16).reshape(-1)), g
        ref = O.channel_decode(ref_codes, ref_ranges, bits, G)
        assert np.array_equal(out[t0:t0 + G].cpu().numpy().view(np.uint32), ref.view(np.uint32)), g
    print(f"config 5 K: {len(picks)} groups bit-exact; every token", flush=True)
    r = ranges.view(groups, 2, D).float()
    lo, hi = r[:, 0], r[:, 1]
    assert bool(torch.isfinite(r).all()) and bool((lo <= hi).all())
    # half a step, the fp16 rounding of the range ends (relative half-ulp 2^-11, absolute 2^-25 below the
    # normal range) and float32 rounding
    step = ((hi - lo) / (2 ** bits - 1)).clamp_min(0)
    tolg = 0.5 * step * (1 + 1e-5) + 4.9e-4 * torch.maximum(lo.abs(), hi.abs()) + 6e-8
    gpl = H * T // G                            # groups per layer
    for layer in range(L):
        a, b = layer * H * T, (layer + 1) * H * T
        assert bool(torch.isfinite(out[a:b]).all()), f"layer {layer}: unwritten or non-finite output"
        tol = tolg[layer * gpl:(layer + 1) * gpl].repeat_interleave(G, 0)
        bad = (x[a:b] - out[a:b]).abs_() > tol
        assert not bool(bad.any()), f"layer {layer}: {int(bad.sum())} elements beyond half a step"
        del tol, bad
    del x, codes, ranges, out, r, lo, hi, step, tolg
    torch.cuda.empty_cache()
