"""GPU tests of the batched decode (pitch_enqueue_decode_batch, PITCH.enqueueDecodeBatch, DecodeBatch).

A batch must write exactly what one enqueueDecode per segment writes, byte for byte, for both methods, every output
element type and a spread of dimensions and bit widths, with ragged segment lengths, segments in separate buffers
and at byte offsets, more segments than one launch takes (32), segments on either side of the length from which a
segment gets a launch of its own (2^18 vectors), mixed with short ones, and a float32 d = 1024 segment long enough
that its single call runs the streaming decoder. A batch with one invalid segment launches nothing. The single-call decoders are pinned against the oracle elsewhere (test_gpu_parity.py);
one case here also checks the batch against the oracle's decode directly (pitch_reference.py:104-107, 123-129).
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O

pytestmark = pytest.mark.gpu


def _segments(torch, dev, d, counts, dtype, seed, cfg):
    """(codes, scales, output, count, codesOffset, scalesOffset, outputOffset) per segment: random code bytes (every
    byte pattern is a valid code stream, unused high bits included) and positive scales at a random vector offset,
    outputs pre-filled with NaN."""
    g = torch.Generator(device=dev).manual_seed(seed)
    segs = []
    for n in counts:
        pad = int(torch.randint(0, 5, (1,), generator=g, device=dev))
        codes = torch.randint(0, 256, ((pad + n) * cfg.codeStride,), generator=g, device=dev,
                              dtype=torch.int32).to(torch.uint8)
        scales = torch.exp(torch.randn(pad + n, generator=g, device=dev))
        out = torch.full((pad + n, d), float("nan"), dtype=dtype, device=dev)
        segs.append((codes, scales, out, n, pad * cfg.codeStride, pad * 4, pad * d * out.element_size()))
    return segs


def _singles(q, segs, cfg):
    outs = []
    for codes, scales, out, n, co, so, oo in segs:
        o2 = out.clone()
        q.enqueueDecode(codes, scales, o2, n, cfg, codesOffset=co, scalesOffset=so, outputOffset=oo)
        outs.append(o2)
    return outs


def _bits_equal(torch, a, b):
    iv = torch.int32 if a.element_size() == 4 else torch.int16
    return torch.equal(a.view(iv), b.view(iv))


CASES = [("turboQuant", 64, 3, "float32"), ("turboQuant", 128, 4, "float32"), ("polarQuant", 128, 4, "float32"),
         ("polarQuant", 64, 5, "float32"), ("turboQuant", 1024, 2, "float32"), ("turboQuant", 256, 8, "float32"),
         ("polarQuant", 512, 3, "float32"), ("turboQuant", 32, 3, "float32"), ("turboQuant", 64, 4, "float16"),
         ("turboQuant", 128, 8, "bfloat16"), ("polarQuant", 64, 2, "float16"), ("turboQuant", 2, 5, "float32"),
         ("polarQuant", 16, 7, "float32"), ("turboQuant", 4, 6, "bfloat16"), ("polarQuant", 1024, 6, "float16")]


@pytest.mark.parametrize("method,d,bits,dtype", CASES)
def test_decode_batch_equals_single_calls(q, method, d, bits, dtype):
    import torch
    import pitch_amd as P
    dev = q.device
    print(f"decode batch {method} d={d} b={bits} {dtype}", flush=True)
    cfg = P.QuantConfig(method, d, bits, 0x1357 + d + bits)
    counts = [8] * 20 + [1, 12, 100, 777, 3, 4096, 8, 8, 9, 31, 64, 65, 200, 5, 2]   # 35 segments: two launches
    segs = _segments(torch, dev, d, counts, getattr(torch, dtype), d * 10 + bits, cfg)
    want = _singles(q, segs, cfg)
    q.enqueueDecodeBatch(segs, cfg)
    torch.cuda.synchronize()
    for i, (seg, o2) in enumerate(zip(segs, want)):
        assert _bits_equal(torch, seg[2], o2), f"segment {i} ({seg[3]} vectors): output differs"


def test_decode_batch_against_oracle(q):
    """A batch's rows against the oracle's decode of the same codes (relative L2 <= 1e-5)."""
    import torch
    import pitch_amd as P
    from test_gpu_parity import REL_L2_BAR, max_rel_diff
    dev = q.device
    for method in ("turboQuant", "polarQuant"):
        cfg = P.QuantConfig(method, 128, 3, 0x2468)
        segs = _segments(torch, dev, 128, [300] * 28, torch.float32, 11, cfg)
        q.enqueueDecodeBatch(segs, cfg)
        torch.cuda.synchronize()
        for codes, scales, out, n, co, so, oo in segs[::9]:
            pad = so // 4
            C = codes[co:co + n * cfg.codeStride].cpu().numpy().tobytes()
            ref = O.DECODERS[method](O.unpack_codes(C, n, 128, 3), scales[pad:pad + n].cpu().numpy().astype(np.float64),
                                     3, cfg.seed)
            assert max_rel_diff(out[pad:pad + n].cpu().numpy(), ref, 128) < REL_L2_BAR


def test_decode_batch_long_segments(q):
    """Segments just below and at 2^18 vectors (the batched kernel, and a launch of their own) between short ones; a
    float32 d = 1024 segment of 2^19 + 17 vectors (whose single call runs the streaming decoder) and a d = 128 one of
    2^22 + 17 decode to the same bytes in the batch."""
    import torch
    import pitch_amd as P
    dev = q.device
    for d, bits, counts in ((2, 4, [(1 << 18) - 1, 5, 1 << 18, 77]), (64, 3, [9, (1 << 18) + 3, (1 << 18) - 2]),
                            (1024, 3, [(1 << 19) + 17, 100]), (128, 3, [(1 << 22) + 17, 100])):
        print(f"decode batch long segments d={d} {counts}", flush=True)
        cfg = P.QuantConfig("turboQuant", d, bits)
        segs = _segments(torch, dev, d, counts, torch.float32, 9 + d, cfg)
        want = _singles(q, segs, cfg)
        q.enqueueDecodeBatch(segs, cfg)
        torch.cuda.synchronize()
        for seg, o2 in zip(segs, want):
            assert _bits_equal(torch, seg[2], o2)
        del segs, want
        torch.cuda.empty_cache()


def test_decode_batch_table_over_layers(q):
    """DecodeBatch over 28 layers' caches (a decode step's per-layer decodes): growing counts and per-segment offsets
    equal single calls."""
    import torch
    import pitch_amd as P
    dev = q.device
    layers, heads, d, T = 28, 2, 128, 40
    cfg = P.QuantConfig("turboQuant", d, 4)
    g = torch.Generator(device=dev).manual_seed(4)
    codes = [torch.randint(0, 256, (T * heads * cfg.codeStride,), generator=g, device=dev,
                           dtype=torch.int32).to(torch.uint8) for _ in range(layers)]
    scales = [torch.rand(T * heads, generator=g, device=dev) + 0.5 for _ in range(layers)]
    outs = [torch.zeros(T * heads, d, device=dev) for _ in range(layers)]
    tab = P.DecodeBatch(q, cfg, codes, scales, outs)
    assert len(tab) == layers
    for t in (1, 17, T):
        tab.enqueue(t * heads)
        torch.cuda.synchronize()
        for l in range(layers):
            ref = torch.zeros_like(outs[l])
            q.enqueueDecode(codes[l], scales[l], ref, t * heads, cfg)
            torch.cuda.synchronize()
            assert _bits_equal(torch, outs[l][:t * heads], ref[:t * heads])
    # one value per segment: each layer decodes its own slice
    first = np.arange(layers, dtype=np.int64) % 5
    tab.enqueue(np.full(layers, 3, np.int64), codesOffsets=first * cfg.codeStride, scalesOffsets=first * 4,
                outputOffsets=np.zeros(layers, np.int64))
    torch.cuda.synchronize()
    for l in range(layers):
        ref = torch.zeros(3, d, device=dev)
        q.enqueueDecode(codes[l], scales[l], ref, 3, cfg, codesOffset=int(first[l]) * cfg.codeStride,
                        scalesOffset=int(first[l]) * 4)
        torch.cuda.synchronize()
        assert _bits_equal(torch, outs[l][:3], ref)
    with pytest.raises(P.InvalidInput):
        tab.enqueue(0)
    with pytest.raises(P.InvalidInput):
        tab.enqueue(1, outputOffsets=-4)


def test_decode_batch_with_an_invalid_segment_launches_nothing(q):
    import torch
    import pitch_amd as P
    dev = q.device
    cfg = P.QuantConfig("turboQuant", 64, 4)
    segs = _segments(torch, dev, 64, [8, 8, 8], torch.float32, 1, cfg)
    codes, scales, out, n, co, so, oo = segs[2]
    bad = (codes, scales, out[:n - 1], n, 0, 0, 0)   # output one vector short
    before = [s[2].clone() for s in segs]
    with pytest.raises(P.InvalidInput, match="output"):
        q.enqueueDecodeBatch(segs[:2] + [bad], cfg)
    torch.cuda.synchronize()
    for s, b in zip(segs, before):
        assert _bits_equal(torch, s[2], b)
    with pytest.raises(P.InvalidInput):
        q.enqueueDecodeBatch([], cfg)
    with pytest.raises(P.InvalidInput):
        q.enqueueDecodeBatch([segs[0], (codes, scales, out.half(), n)], cfg)   # mixed element types
