"""GPU tests of the batched encode (pitch_enqueue_encode_batch, PITCH.enqueueEncodeBatch, EncodeBatch).

A batch must write exactly what one enqueueEncode per segment writes (codes and scales bit for bit: it runs the
encoder a single call of its configuration runs), for every method, element type and a spread of dimensions and
bit widths, with ragged segment lengths, segments in separate buffers and at byte offsets, more segments than one
launch takes (32), and a segment long enough to loop over its rounds. A batch with one invalid segment launches nothing. The single-call encoders are pinned
against the oracle elsewhere (test_gpu_parity.py); one case here also checks sampled rows against the oracle
directly (pitch_reference.py:92-121).
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import check_codes, check_scales

pytestmark = pytest.mark.gpu


def _segments(torch, dev, d, counts, dtype, seed, cfg):
    g = torch.Generator(device=dev).manual_seed(seed)
    segs = []
    for n in counts:
        pad = int(torch.randint(0, 5, (1,), generator=g, device=dev))  # vectors of offset before the segment
        x = torch.randn(pad + n, d, generator=g, device=dev) * torch.exp(torch.randn(pad + n, 1, generator=g,
                                                                                     device=dev))
        x = x.to(dtype)
        codes = torch.full(((pad + n) * cfg.codeStride,), 0xA5, dtype=torch.uint8, device=dev)
        scales = torch.full((pad + n,), -1.0, device=dev)
        segs.append((x, codes, scales, n, pad * d * x.element_size(), pad * cfg.codeStride, pad * 4))
    return segs


def _singles(q, segs, cfg, torch):
    out = []
    for x, codes, scales, n, io, co, so in segs:
        c2, s2 = codes.clone(), scales.clone()
        q.enqueueEncode(x, c2, s2, n, cfg, inputOffset=io, codesOffset=co, scalesOffset=so)
        out.append((c2, s2))
    return out


# Every encoder a single call can run, so every batched form: the staged-stage encoder (float32, d = 64 / 128),
# the LDS-transposed one (float32, d >= 256; b = 8 has the densest decision edges), the lane-per-vector
# TurboQuant encoder (float32 d = 8 .. 32, 16-bit d = 64 / 128) and the team encoder (the rest).
CASES = [("turboQuant", 64, 3, "float32"), ("turboQuant", 128, 4, "float32"), ("polarQuant", 128, 4, "float32"),
         ("polarQuant", 64, 5, "float32"),
         ("turboQuant", 1024, 2, "float32"), ("turboQuant", 256, 8, "float32"), ("polarQuant", 512, 3, "float32"),
         ("turboQuant", 32, 3, "float32"), ("turboQuant", 64, 4, "float16"), ("turboQuant", 128, 8, "bfloat16"),
         ("polarQuant", 64, 2, "float16"), ("turboQuant", 2, 5, "float32"), ("polarQuant", 16, 7, "float32"),
         ("turboQuant", 256, 3, "float16"), ("polarQuant", 512, 6, "bfloat16")]


@pytest.mark.parametrize("method,d,bits,dtype", CASES)
def test_batch_equals_single_calls(q, method, d, bits, dtype):
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"batch {method} d={d} b={bits} {dtype}", flush=True)
    cfg = P.QuantConfig(method, d, bits, 0x2468 + d + bits)
    counts = [8] * 20 + [1, 12, 100, 777, 3, 4096, 8, 8, 9, 31, 64, 65, 200, 5, 2]   # 35 segments: two launches
    segs = _segments(torch, dev, d, counts, getattr(torch, dtype), d * 10 + bits, cfg)
    want = _singles(q, segs, cfg, torch)
    q.enqueueEncodeBatch(segs, cfg)
    torch.cuda.synchronize()
    for i, ((x, codes, scales, n, _, _, _), (c2, s2)) in enumerate(zip(segs, want)):
        assert torch.equal(codes, c2), f"segment {i} ({n} vectors): codes differ"
        assert torch.equal(scales.view(torch.int32), s2.view(torch.int32)), f"segment {i}: scales differ"


def test_batch_against_oracle(q):
    """Sampled rows of a batch against the oracle's encode (codes except at near-boundary coordinates, scales
    within one float32 ulp)."""
    import torch
    import pitch_amd as P
    dev = q.device
    cfg = P.QuantConfig("turboQuant", 128, 3, 0x1357)
    segs = _segments(torch, dev, 128, [8] * 32, torch.float32, 5, cfg)
    q.enqueueEncodeBatch(segs, cfg)
    torch.cuda.synchronize()
    for x, codes, scales, n, io, co, so in segs[::7]:
        pad = so // 4
        X = x[pad:pad + n].cpu().numpy()
        ref_c, ref_s = O.turbo_encode(X.astype(np.float64), 3, cfg.seed)
        ours = codes[co:co + n * cfg.codeStride].cpu().numpy().tobytes()
        check_codes("turboQuant", X, 3, cfg.seed, ours, O.pack_codes(ref_c, 3), "batch")
        check_scales(scales[pad:pad + n].cpu().numpy(), ref_s, "batch")


def test_batch_long_segment_loops(q):
    """A segment longer than 1024 workgroups' rounds is covered by its workgroups' loop."""
    import torch
    import pitch_amd as P
    dev = q.device
    cfg = P.QuantConfig("turboQuant", 2, 4)
    n = 300_000 + 77
    segs = _segments(torch, dev, 2, [n, 5], torch.float32, 9, cfg)
    want = _singles(q, segs, cfg, torch)
    q.enqueueEncodeBatch(segs, cfg)
    torch.cuda.synchronize()
    for (x, codes, scales, *_), (c2, s2) in zip(segs, want):
        assert torch.equal(codes, c2) and torch.equal(scales.view(torch.int32), s2.view(torch.int32))


def test_encode_batch_table_appends_tokens(q):
    """EncodeBatch over 32 layers' caches: per-token appends at advancing offsets equal single calls."""
    import torch
    import pitch_amd as P
    dev = q.device
    layers, heads, d, T = 32, 8, 128, 5
    cfg = P.QuantConfig("turboQuant", d, 3)
    g = torch.Generator(device=dev).manual_seed(3)
    new = [torch.randn(T, heads, d, generator=g, device=dev) for _ in range(layers)]
    caches = [(torch.zeros(T * heads * cfg.codeStride, dtype=torch.uint8, device=dev),
               torch.zeros(T * heads, device=dev)) for _ in range(layers)]
    tab = P.EncodeBatch(q, cfg, new, [c for c, _ in caches], [s for _, s in caches])
    assert len(tab) == layers
    for t in range(T):
        tab.enqueue(heads, inputOffsets=t * heads * d * 4, codesOffsets=t * heads * cfg.codeStride,
                    scalesOffsets=t * heads * 4)
    ref = [(torch.zeros_like(c), torch.zeros_like(s)) for c, s in caches]
    for l in range(layers):
        q.enqueueEncode(new[l], ref[l][0], ref[l][1], T * heads, cfg)
    torch.cuda.synchronize()
    for (c, s), (rc, rs) in zip(caches, ref):
        assert torch.equal(c, rc) and torch.equal(s.view(torch.int32), rs.view(torch.int32))
    # per-segment counts and offsets
    tab.enqueue(np.full(layers, 3, np.int64), codesOffsets=np.zeros(layers, np.int64))
    with pytest.raises(P.InvalidInput):
        tab.enqueue(0)
    with pytest.raises(P.InvalidInput):
        tab.enqueue(1, codesOffsets=-4)


def test_batch_with_an_invalid_segment_launches_nothing(q):
    import torch
    import pitch_amd as P
    dev = q.device
    cfg = P.QuantConfig("turboQuant", 64, 4)
    segs = _segments(torch, dev, 64, [8, 8, 8], torch.float32, 1, cfg)
    x, codes, scales, n, io, co, so = segs[2]
    bad = (x, codes[:n * cfg.codeStride - 4], scales, n, 0, 0, 0)   # codes 4 bytes short
    before = [s[1].clone() for s in segs]
    with pytest.raises(P.InvalidInput, match="codes"):
        q.enqueueEncodeBatch(segs[:2] + [bad], cfg)
    torch.cuda.synchronize()
    for s, b in zip(segs, before):
        assert torch.equal(s[1], b)
    with pytest.raises(P.InvalidInput):
        q.enqueueEncodeBatch([], cfg)
    with pytest.raises(P.InvalidInput):
        q.enqueueEncodeBatch([segs[0], (x.half(), codes, scales, n)], cfg)   # mixed element types
