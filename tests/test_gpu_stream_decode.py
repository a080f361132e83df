"""GPU parity of long float32 decodes: at d = 1024 the streaming decoder (calls of at least 2^19 vectors; one launch
held at 5 workgroups per CU for codes of up to 6 bits, launches of one round for 7 and 8), at d = 128 `vec_decode`
with one workgroup per block (2^22 vectors here: the same 2 GB of output).

Codes are random bytes (at d = 128 and 1024 every bit width packs into whole words, so any byte pattern is a valid
code stream) with random positive scales. One call of the threshold + 4099 vectors (a ragged last launch) per
dimension, method and bit width is checked:
* sampled rows against the oracle's decode of the same codes: relative L2 <= 1e-5 (pitch_reference.py:104-107,
  123-129);
* the first and last 65536 vectors against the persistent decoder (separate calls below the streaming size, through
  byte offsets): byte for byte, so a slice decoded at an offset equals the same rows of a whole-cache decode (both
  decoders run the butterflies in the same bit order and give exact zeros the sign +0 before the rotation signs);
* every output element written (pre-filled with NaN) and finite.
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O
from test_gpu_parity import max_rel_diff, REL_L2_BAR

pytestmark = pytest.mark.gpu

@pytest.mark.parametrize("D", [128, 1024])
@pytest.mark.parametrize("method", ["turboQuant", "polarQuant"])
@pytest.mark.parametrize("bits", [2, 3, 4, 5, 6, 7, 8])
def test_stream_decode(q, D, method, bits):
    import torch
    import pitch_amd as P
    dev = q.device
    N = ((1 << 22) * 128 // D) + 4099
    print(f"streaming decode d={D} {method} b={bits} n={N}", flush=True)
    cfg = P.QuantConfig(method, D, bits, 0x1234 + bits)
    g = torch.Generator(device=dev).manual_seed(900 + bits + (method == "polarQuant"))
    codes = torch.randint(0, 256, (N * cfg.codeStride,), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    scales = torch.exp(torch.randn(N, generator=g, device=dev))
    out = torch.full((N, D), float("nan"), device=dev)
    q.enqueueDecode(codes, scales, out, N, cfg)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    rng = np.random.default_rng(bits)
    idx = np.unique(np.concatenate([np.arange(64), np.arange(N - 64, N), rng.integers(0, N, 512)]))
    it = torch.from_numpy(idx).to(dev)
    C = codes.view(N, cfg.codeStride)[it].cpu().numpy().tobytes()
    S = scales[it].cpu().numpy().astype(np.float64)
    ref = O.DECODERS[method](O.unpack_codes(C, len(idx), D, bits), S, bits, cfg.seed)
    assert max_rel_diff(out[it].cpu().numpy(), ref, D) < REL_L2_BAR
    m = 65536
    for v0 in (0, N - m):
        part = torch.empty(m, D, device=dev)
        q.enqueueDecode(codes, scales, part, m, cfg, codesOffset=v0 * cfg.codeStride, scalesOffset=v0 * 4)
        torch.cuda.synchronize()
        differ = int((out[v0:v0 + m].view(torch.int32) != part.view(torch.int32)).sum())
        assert differ == 0, (v0, differ)
    del codes, scales, out
    torch.cuda.empty_cache()
