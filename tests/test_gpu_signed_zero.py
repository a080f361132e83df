"""KIVI ranges when a channel's extreme is zero: the fp16 range bits must equal the reference's.

The reference takes per-group channel minima and maxima with numpy (pitch_reference.py:150-153), whose min / max keep
the LAST of equal values in token order, so an extreme of zero carries the sign of the channel's last zero
(tests/test_oracle_known.py pins that numpy behaviour). The kernels reduce in other orders and fix such extremes up;
this test places zeros of both signs, in varied orders, at the minimum, the maximum and in all-zero channels, for
every per-channel encoder (the wave encoder at G <= 64 and d % 4 == 0, the 4-channel encoder at larger G, the
1-channel encoder at d % 4 != 0) and for 16-bit keys, and compares codes and range bits with the oracle.
"""
import numpy as np
import pytest

from oracle import pitch_oracle as O

pytestmark = pytest.mark.gpu


def _keys(n, d, seed):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((n, d)).astype(np.float32)
    for c in range(d):
        kind = c % 5
        zpos = rng.choice(n, size=min(n, 1 + c % 7), replace=False)
        zeros = np.where(rng.random(len(zpos)) < 0.5, np.float32(-0.0), np.float32(0.0))
        if kind == 0:      # minimum is zero: non-negative channel
            X[:, c] = np.abs(X[:, c]) + 0.5
        elif kind == 1:    # maximum is zero: non-positive channel
            X[:, c] = -np.abs(X[:, c]) - 0.5
        elif kind == 2:    # all zeros, mixed signs
            X[:, c] = np.where(rng.random(n) < 0.5, np.float32(-0.0), np.float32(0.0))
            continue
        elif kind == 3:    # zeros strictly inside the range: no effect on the extremes
            pass
        else:              # a single-signed zero run at the very end
            X[:, c] = np.abs(X[:, c]) + 0.25
            zpos = np.array([n - 1])
            zeros = np.array([np.float32(-0.0) if c % 2 else np.float32(0.0)])
        X[zpos, c] = zeros
    return X


@pytest.mark.parametrize("n,d,G", [(150, 64, 64), (150, 64, 16), (130, 96, 32), (300, 64, 100), (50, 7, 16),
                                   (70, 12, 128)])
@pytest.mark.parametrize("io", ["float32", "float16", "bfloat16"])
def test_zero_extremes_take_the_last_zeros_sign(q, n, d, G, io):
    import torch
    import pitch_amd as P
    print(f"signed-zero extremes n={n} d={d} G={G} io={io}", flush=True)
    X = _keys(n, d, n + d + G)
    t = torch.from_numpy(X).to(q.device).to(getattr(torch, io))
    Xw = t.float().cpu().numpy()                 # the keys as the kernel widens them (exact)
    cfg = P.ChannelQuantConfig(d, 4, G)
    groups = cfg.groupCount(n)
    codes = torch.zeros(n * cfg.codeStride, dtype=torch.uint8, device=q.device)
    ranges = torch.zeros(groups * 2 * d, dtype=torch.float16, device=q.device)
    q.enqueuePerChannelEncode(t, codes, ranges, n, cfg)
    torch.cuda.synchronize()
    ref_codes, ref_ranges = O.channel_encode(Xw, 4, G)
    got = ranges.cpu().numpy().view(np.uint16).reshape(groups, 2, d)
    want = ref_ranges.view(np.uint16)
    bad = np.argwhere(got != want)
    assert not len(bad), f"range bits differ at (group, lo/hi, channel) {bad[:5].tolist()}: " \
                         f"{got[tuple(bad[0])]:#06x} vs {want[tuple(bad[0])]:#06x}"
    assert codes.cpu().numpy().tobytes() == O.pack_codes(ref_codes, 4)
    # the case the test exists for occurs
    assert (want == 0x8000).any() and (want == 0x0000).any()
