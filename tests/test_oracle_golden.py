"""The CPU oracle against the reference's golden vectors (CPU only).

* parity.json (40 per-vector cases) and channel_parity.json (17 KIVI cases): the reference's fixtures,
  written by reference/gen_fixtures.py:63-148 and checked by ParityTests.metalMatchesReference
  (Tests/PITCHTests/ParityTests.swift:48-83) and PerChannelTests.metalMatchesReference
  (Tests/PITCHTests/PerChannelTests.swift:66-98);
* ref_vectors.npz: vectors written from reference/pitch_reference.py at the shapes the fixtures leave open
  (d in {4, 8, 32, 128, 512}, bits 5..7, KIVI dims {1, 7, 33, 64, 128} and group sizes {1, 16, 64, 100});
* BASELINE config 1 (4096 x 64 N(0,1), rotation seed 1, b = 4): codes, norms and reconstruction hash.

The oracle must reproduce packed codes, float32 scales, fp16 ranges and KIVI reconstructions bit for bit, and
the per-vector reconstructions to float64 rounding noise (they are float64 sums cast to float32).
"""
import base64
import hashlib

import numpy as np
import pytest

import golden_data as gd
from oracle import pitch_oracle as O

PV_RECON_TOL = 1e-12      # per-vector relative L2 of the float32 reconstruction vs the reference's
PV_CASES = gd.parity()[1]
CH_CASES = gd.channel_parity()[1]


def _rel_l2(a, b):
    a = np.asarray(a, np.float64).reshape(b.shape[0], -1)
    b = np.asarray(b, np.float64).reshape(b.shape[0], -1)
    den = np.sqrt((b ** 2).sum(1))
    return float(np.max(np.sqrt(((a - b) ** 2).sum(1)) / np.where(den > 0, den, 1.0)))


def test_fixture_completeness():
    """ParityTests.swift:42-46 and PerChannelTests.swift:60-64: 40 and 17 cases."""
    groups, cases = gd.parity()
    assert len(cases) == 40
    assert {(c["group"], c["method"], c["bits"]) for c in cases} == {
        (g, m, b) for g in groups for m in ("turboQuant", "polarQuant") for b in (2, 3, 4, 8)}
    assert len(CH_CASES) == 17


def per_vector_check(X, method, bits, seed, codes_ref: bytes, scales_ref, recon_ref):
    codes, scales = O.ENCODERS[method](X.astype(np.float64), bits, seed)
    assert O.pack_codes(codes, bits) == codes_ref, "packed codes differ"
    s32 = np.asarray(scales, np.float32)
    assert np.array_equal(s32.view(np.uint32), np.asarray(scales_ref, np.float32).view(np.uint32)), "scales differ"
    recon = O.DECODERS[method](codes, s32.astype(np.float64), bits, seed).astype(np.float32)
    ref = np.asarray(recon_ref, np.float32).reshape(recon.shape)
    assert _rel_l2(recon, ref) <= PV_RECON_TOL
    return recon


@pytest.mark.parametrize("i", range(len(PV_CASES)))
def test_parity_fixture(i):
    groups, cases = gd.parity()
    c = cases[i]
    X = groups[c["group"]]
    recon = per_vector_check(X, c["method"], c["bits"], c["seed"], base64.b64decode(c["codes"]),
                             gd.f32(c["scales"]), gd.f32(c["reconstruction"]))
    # the fixture's relative_error (reference/gen_fixtures.py:90) from the oracle's own reconstruction
    Xd = X.astype(np.float64)
    rel = float((((Xd - recon.astype(np.float64)) ** 2).sum(1) / (Xd ** 2).sum(1)).mean())
    assert rel == pytest.approx(c["relative_error"], rel=1e-5)


@pytest.mark.parametrize("i", range(len(CH_CASES)))
def test_channel_fixture(i):
    groups, cases = gd.channel_parity()
    c = cases[i]
    X = groups[c["group"]]
    codes, ranges = O.channel_encode(X, c["bits"], c["group_size"])
    assert O.pack_codes(codes, c["bits"]) == base64.b64decode(c["codes"])
    assert np.array_equal(ranges.view(np.uint16).reshape(-1), gd.u16(c["ranges"]))
    recon = O.channel_decode(codes, ranges, c["bits"], c["group_size"])
    assert np.array_equal(recon.reshape(-1).view(np.uint32), gd.f32(c["reconstruction"]).view(np.uint32))
    mse = float(((X.astype(np.float64) - recon) ** 2).mean())
    assert mse == pytest.approx(c["mse"], rel=1e-9)


def test_ref_vectors_per_vector():
    cases = gd.ref_per_vector_cases()
    assert len(cases) >= 150
    dims = {X.shape[1] for _, X, *_ in cases}
    assert {4, 8, 32, 128, 512} <= dims
    assert {b for _, _, _, b, *_ in cases} == set(range(2, 9))
    for key, X, method, bits, seed, codes, scales, recon in cases:
        try:
            per_vector_check(X, method, bits, seed, codes, scales, recon)
        except AssertionError as e:
            raise AssertionError(f"{key}: {e}") from None


def test_ref_vectors_per_channel():
    cases = gd.ref_channel_cases()
    assert len(cases) >= 50
    for key, X, bits, G, codes_ref, ranges_ref, recon_ref in cases:
        codes, ranges = O.channel_encode(X, bits, G)
        assert O.pack_codes(codes, bits) == codes_ref, key
        assert np.array_equal(ranges.view(np.uint16).reshape(-1), np.asarray(ranges_ref).reshape(-1)), key
        recon = O.channel_decode(codes, ranges, bits, G)
        assert np.array_equal(recon.view(np.uint32).reshape(-1),
                              np.asarray(recon_ref, np.float32).view(np.uint32).reshape(-1)), key


def test_config1():
    """BASELINE config 1 through the oracle: codes and norms as written by the reference, reconstruction hash."""
    z = gd.ref_vectors()
    X = gd.config1_inputs()
    assert hashlib.sha256(X.tobytes()).digest() == z["cfg1/input_sha256"].tobytes(), "numpy stream changed"
    codes, norms = O.turbo_encode(X.astype(np.float64), 4, 1)
    assert O.pack_codes(codes, 4) == z["cfg1/codes"].tobytes()
    n32 = norms.astype(np.float32)
    assert np.array_equal(n32.view(np.uint32), z["cfg1/scales"].view(np.uint32))
    recon = O.turbo_decode(codes, n32.astype(np.float64), 4, 1).astype(np.float32)
    assert hashlib.sha256(recon.tobytes()).digest() == z["cfg1/recon_sha256"].tobytes()
