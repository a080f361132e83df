"""GPU tests of the cache-maintenance entry points around the codec kernels.

* pitch_enqueue_channel_append: a per-channel key cache grown token by token (and in ragged batches) holds,
  after every append, exactly what one encode of all its tokens gives, which the oracle fixes bit for bit:
  complete groups keep their ranges and a partial last group is re-encoded over the tokens it holds
  (README.md:85; oracle.channel_encode of the prefix, reference/pitch_reference.py:145-162).
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d,G,bits,io", [(64, 64, 4, "float32"), (128, 32, 3, "float16"), (33, 8, 5, "bfloat16"),
                                         (96, 128, 2, "float32")])
def test_channel_append_matches_encode_of_prefix(q, d, G, bits, io):
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"append d={d} G={G} b={bits} {io}", flush=True)
    rng = np.random.default_rng(d + G + bits)
    steps = [1, 1, 5, G - 1, 1, 2 * G + 3, 1, G, 17]
    T = sum(steps)
    X = (rng.standard_normal((T, d)) * np.exp(rng.standard_normal(d)) + 2 * rng.standard_normal(d))
    x = torch.from_numpy(X.astype(np.float32)).to(dev).to(getattr(torch, io)).contiguous()
    Xw = x.float().cpu().numpy()                      # the widened values the kernels see
    cfg = P.ChannelQuantConfig(d, bits, G)
    codes = torch.zeros(T * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.zeros(cfg.groupCount(T) * 2 * d, dtype=torch.float16, device=dev)
    total = 0
    for n in steps:
        total += n
        q.enqueuePerChannelAppend(x, codes, ranges, total, n, cfg)
        torch.cuda.synchronize()
        ref_codes, ref_ranges = O.channel_encode(Xw[:total], bits, G)
        got = codes[:total * cfg.codeStride].cpu().numpy().tobytes()
        assert got == O.pack_codes(ref_codes, bits), (total, n)
        g = cfg.groupCount(total)
        got_r = ranges[:g * 2 * d].cpu().numpy().view(np.uint16)
        assert np.array_equal(got_r, ref_ranges.view(np.uint16).reshape(-1)), (total, n)
    out = torch.empty(T, d, dtype=torch.float32, device=dev)
    q.enqueuePerChannelDecode(codes, ranges, out, T, cfg)
    torch.cuda.synchronize()
    ref = O.channel_decode(*O.channel_encode(Xw, bits, G), bits, G)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def _rope(positions, d, dev):
    import torch
    inv = 1.0 / 1e6 ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(positions, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat([torch.cos(ang)] * 2, 1).float().to(dev).contiguous()
    sin = torch.cat([torch.sin(ang)] * 2, 1).float().to(dev).contiguous()
    return cos, sin


@pytest.mark.parametrize("method,d,bits", [("turboQuant", 64, 4), ("turboQuant", 128, 3), ("polarQuant", 128, 4),
                                           ("turboQuant", 256, 2), ("turboQuant", 2, 4), ("polarQuant", 8, 5)])
def test_key_bias_removal(q, method, d, bits):
    """Encoding with the RoPE'd key bias removed equals encoding x - R_t b (computed by torch in float32 in the
    reference's order) byte for byte, meets the oracle on those vectors, and the decode adds R_t b back."""
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"key bias {method} d={d} b={bits}", flush=True)
    heads, T, first = 4, 301, 37
    n = heads * T
    g = torch.Generator(device=dev).manual_seed(d + bits)
    bias = (torch.randn(heads, d, generator=g, device=dev) * 8).contiguous()
    cos, sin = _rope(first + T + 5, d, dev)
    t = first + torch.arange(n, device=dev) // heads
    h = torch.arange(n, device=dev) % heads
    bb = bias[h]
    rh = torch.cat([-bb[:, d // 2:], bb[:, :d // 2]], 1)
    o = bb * cos[t] + rh * sin[t]                          # R_t b, float32, as mechanism_eval.py:97
    x = (torch.randn(n, d, generator=g, device=dev) + o).contiguous()
    cfg = P.QuantConfig(method, d, bits)
    kb = P.KeyBias(bias, cos, sin, firstPosition=first, heads=heads)
    c1 = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    s1 = torch.empty(n, device=dev)
    c2, s2 = torch.empty_like(c1), torch.empty_like(s1)
    q.enqueueEncode(x, c1, s1, n, cfg, keyBias=kb)
    q.enqueueEncode((x - o).contiguous(), c2, s2, n, cfg)
    out = torch.empty(n, d, device=dev)
    plain = torch.empty(n, d, device=dev)
    q.enqueueDecode(c1, s1, out, n, cfg, keyBias=kb)
    q.enqueueDecode(c1, s1, plain, n, cfg)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2) and torch.equal(s1, s2)
    assert torch.equal(out, plain + o)
    X = x.cpu().numpy()
    Ob = O.key_bias_offsets(bias.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), first, n, heads)
    assert np.array_equal(Ob, o.cpu().numpy())
    Y = (X - Ob).astype(np.float32)
    from test_gpu_parity import check_codes, check_scales, max_rel_diff
    ref_codes, ref_scales = O.ENCODERS[method](Y.astype(np.float64), bits)
    check_codes(method, Y, bits, P.DEFAULT_SEED, c1.cpu().numpy().tobytes(), O.pack_codes(ref_codes, bits),
                f"key bias {method} d={d}")
    check_scales(s1.cpu().numpy(), np.asarray(ref_scales, np.float32), "key bias scales")
    ours = O.unpack_codes(c1.cpu().numpy().tobytes(), n, d, bits)
    ref = O.DECODERS[method](ours, s1.cpu().numpy().astype(np.float64), bits) + Ob
    assert max_rel_diff(out.cpu().numpy(), ref, d) < 1e-5
