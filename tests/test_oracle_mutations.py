"""Planted mistakes in the CPU oracle must be caught by the checks that pin it (CPU only).

Each case patches one plausible slip into the oracle (a flipped sign, a dropped FWHT stage, ties sent to the
upper code, a missing rounding offset, swapped atan2 operands, float32 instead of fp16 ranges, a dropped
straddling bit, ...) and asserts that the golden-vector or known-answer checks then fail. This shows the
checks are strong enough to catch such mistakes in the oracle, and therefore in the kernels compared with it.
"""
import base64
import math

import numpy as np
import pytest

import golden_data as gd
from oracle import pitch_oracle as O

from test_oracle_golden import per_vector_check
from test_oracle_known import edge_straddle_check


def _all_per_vector_fixtures():
    groups, cases = gd.parity()
    for c in cases:
        per_vector_check(groups[c["group"]], c["method"], c["bits"], c["seed"], base64.b64decode(c["codes"]),
                         gd.f32(c["scales"]), gd.f32(c["reconstruction"]))


def _all_channel_fixtures():
    groups, cases = gd.channel_parity()
    for c in cases:
        X = groups[c["group"]]
        codes, ranges = O.channel_encode(X, c["bits"], c["group_size"])
        assert O.pack_codes(codes, c["bits"]) == base64.b64decode(c["codes"])
        assert np.array_equal(ranges.view(np.uint16).reshape(-1), gd.u16(c["ranges"]))
        recon = O.channel_decode(codes, ranges, c["bits"], c["group_size"])
        assert np.array_equal(recon.reshape(-1).view(np.uint32), gd.f32(c["reconstruction"]).view(np.uint32))


def _zero_vector_ties():
    codes, norms = O.turbo_encode(np.zeros((1, 64)), 4)
    assert np.all(codes == 7)


def _constant_channel():
    X = np.random.default_rng(5).standard_normal((64, 8)).astype(np.float32)
    X[:, 0] = 1.5
    codes, ranges = O.channel_encode(X, 2)
    assert np.all(O.channel_decode(codes, ranges, 2)[:, 0] == 1.5)


# ----------------------------------------------------------------------------- mutations
def _signs_negated(monkeypatch):
    orig = O.rand_signs
    monkeypatch.setattr(O, "rand_signs", lambda seed, d: -orig(seed, d))


def _wht_last_stage_dropped(monkeypatch):
    def wht(x):
        x = np.array(x, dtype=np.float64, copy=True)
        n, d = x.shape
        h = 1
        while 2 * h < d:
            v = x.reshape(n, d // (2 * h), 2, h)
            a, b = v[:, :, 0, :].copy(), v[:, :, 1, :].copy()
            v[:, :, 0, :], v[:, :, 1, :] = a + b, a - b
            h *= 2
        return x
    monkeypatch.setattr(O, "wht", wht)


def _ties_to_upper_code(monkeypatch):
    def turbo_encode(X, b, seed=O.DEFAULT_SEED):
        X = np.asarray(X, dtype=np.float64)
        norms = np.linalg.norm(X, axis=1)
        U = O.rotate(X / np.where(norms > 0, norms, 1.0)[:, None], seed)
        return np.searchsorted(O.turbo_edges(X.shape[1], b), U, side="right"), norms
    monkeypatch.setattr(O, "turbo_encode", turbo_encode)
    monkeypatch.setitem(O.ENCODERS, "turboQuant", turbo_encode)


def _no_sqrt_d_in_unrotate(monkeypatch):
    monkeypatch.setattr(O, "unrotate", lambda Y, seed: O.wht(Y) * O.rand_signs(seed, Y.shape[1]))


def _polar_no_half(monkeypatch):
    def polar_encode(X, b, seed=O.DEFAULT_SEED):
        r, theta = O.polar_parts(X, seed)
        RL, N = 2 ** b - 1, 2 ** b
        rmax = r.max(axis=1)
        safe = np.where(rmax > 0, rmax, 1.0)[:, None]
        codes = np.empty((r.shape[0], 2 * r.shape[1]), dtype=np.int64)
        codes[:, 0::2] = np.clip(np.floor(r / safe * RL), 0, RL)
        codes[:, 1::2] = np.mod(np.floor(theta / (2 * np.pi) * N + 0.5), N)
        return codes, rmax
    monkeypatch.setattr(O, "polar_encode", polar_encode)
    monkeypatch.setitem(O.ENCODERS, "polarQuant", polar_encode)


def _polar_atan2_swapped(monkeypatch):
    def polar_parts(X, seed=O.DEFAULT_SEED):
        Y = O.rotate(np.asarray(X, dtype=np.float64), seed)
        a, c = Y[:, 0::2], Y[:, 1::2]
        return np.hypot(a, c), np.mod(np.arctan2(a, c), 2 * np.pi)
    monkeypatch.setattr(O, "polar_parts", polar_parts)


def _polar_decode_cos_sin_swapped(monkeypatch):
    def polar_decode(codes, rmax, b, seed=O.DEFAULT_SEED):
        RL, N = 2 ** b - 1, 2 ** b
        r = codes[:, 0::2] / RL * np.asarray(rmax, dtype=np.float64)[:, None]
        theta = codes[:, 1::2] / N * 2 * np.pi
        Y = np.empty(codes.shape)
        Y[:, 0::2], Y[:, 1::2] = r * np.sin(theta), r * np.cos(theta)
        return O.unrotate(Y, seed)
    monkeypatch.setattr(O, "polar_decode", polar_decode)
    monkeypatch.setitem(O.DECODERS, "polarQuant", polar_decode)


def _edges_in_float64(monkeypatch):
    monkeypatch.setattr(O, "turbo_edges", lambda d, b: 0.5 * (O.turbo_codebook(d, b)[1:]
                                                              + O.turbo_codebook(d, b)[:-1]))


def _kivi_float32_ranges(monkeypatch):
    orig = O.channel_encode

    def channel_encode(X, b, G=O.CHANNEL_DEFAULT_GROUP):
        X = np.asarray(X, dtype=np.float32)
        n, d = X.shape
        L = np.float32(2 ** b - 1)
        codes, ranges = orig(X, b, G)
        for g, s in enumerate(range(0, n, G)):
            blk = X[s:s + G]
            lo, hi = blk.min(0), blk.max(0)
            step = (hi - lo) / L
            step[step == 0] = np.float32(1)
            codes[s:s + G] = np.clip(np.floor((blk - lo) / step + np.float32(0.5)), 0, L)
        return codes, ranges
    monkeypatch.setattr(O, "channel_encode", channel_encode)


def _kivi_zero_step_kept(monkeypatch):
    """Encode divides by a zero step for a constant channel instead of by 1."""
    orig = O.channel_encode

    def channel_encode(X, b, G=O.CHANNEL_DEFAULT_GROUP):
        X = np.asarray(X, dtype=np.float32)
        n, d = X.shape
        L = np.float32(2 ** b - 1)
        codes, ranges = orig(X, b, G)
        with np.errstate(divide="ignore", invalid="ignore"):
            for g, s in enumerate(range(0, n, G)):
                lo = ranges[g, 0].astype(np.float32)
                step = (ranges[g, 1].astype(np.float32) - lo) / L
                q = np.floor((X[s:s + G] - lo) / step + np.float32(0.5))
                codes[s:s + G] = np.clip(np.nan_to_num(q, nan=L), 0, L)
        return codes, ranges
    monkeypatch.setattr(O, "channel_encode", channel_encode)


def _kivi_fma_decode(monkeypatch):
    def channel_decode(codes, ranges, b, G=O.CHANNEL_DEFAULT_GROUP):
        n, d = codes.shape
        L = np.float32(2 ** b - 1)
        out = np.empty((n, d), dtype=np.float32)
        for g, s in enumerate(range(0, n, G)):
            lo = ranges[g, 0].astype(np.float32)
            step = (ranges[g, 1].astype(np.float32) - lo) / L
            step[step == 0] = np.float32(1)
            # fused multiply-add: one rounding instead of two
            out[s:s + G] = (codes[s:s + G].astype(np.float64) * step.astype(np.float64)
                            + lo.astype(np.float64)).astype(np.float32)
        return out
    monkeypatch.setattr(O, "channel_decode", channel_decode)


def _pack_drops_straddle(monkeypatch):
    def pack_codes(codes, b):
        codes = np.asarray(codes)
        n, d = codes.shape
        out = np.zeros((n, O.code_stride_bytes(d, b) // 4), dtype=np.uint64)
        c = codes.astype(np.uint64) & np.uint64((1 << b) - 1)
        for i in range(d):
            w, off = (i * b) >> 5, (i * b) & 31
            out[:, w] |= (c[:, i] << np.uint64(off)) & np.uint64(0xFFFFFFFF)
        return out.astype("<u4").tobytes()
    monkeypatch.setattr(O, "pack_codes", pack_codes)


def _scales_not_cast(monkeypatch):
    """Decode with the float64 norms instead of the stored float32 scales (reference/gen_fixtures.py:88-89)."""
    orig = O.turbo_decode
    monkeypatch.setitem(O.DECODERS, "turboQuant",
                        lambda codes, norms, b, seed=O.DEFAULT_SEED: orig(codes, norms * (1 + 2 ** -30), b, seed))


MUTATIONS = {
    "signs negated": (_signs_negated, _all_per_vector_fixtures),
    "last FWHT stage dropped": (_wht_last_stage_dropped, _all_per_vector_fixtures),
    "ties to the upper code": (_ties_to_upper_code, _zero_vector_ties),
    "unrotate without 1/sqrt(d)": (_no_sqrt_d_in_unrotate, _all_per_vector_fixtures),
    "polar radius without +0.5": (_polar_no_half, _all_per_vector_fixtures),
    "polar atan2 operands swapped": (_polar_atan2_swapped, _all_per_vector_fixtures),
    "polar decode cos/sin swapped": (_polar_decode_cos_sin_swapped, _all_per_vector_fixtures),
    "TurboQuant edges in float64": (_edges_in_float64, edge_straddle_check),
    "KIVI codes from float32 ranges": (_kivi_float32_ranges, _all_channel_fixtures),
    "KIVI zero step kept": (_kivi_zero_step_kept, _constant_channel),
    "KIVI decode fused": (_kivi_fma_decode, _all_channel_fixtures),
    "straddling code bits dropped": (_pack_drops_straddle, _all_per_vector_fixtures),
    "decode scale off by 2^-30": (_scales_not_cast, _all_per_vector_fixtures),
}


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_mistake_is_caught(name, monkeypatch):
    plant, check = MUTATIONS[name]
    check()                                  # passes on the real oracle
    plant(monkeypatch)
    with pytest.raises(AssertionError):
        check()


def test_unmutated_checks_pass():
    _all_per_vector_fixtures()
    _all_channel_fixtures()
    _zero_vector_ties()
    _constant_channel()
    assert math.isclose(O.bits_per_coordinate(64, 4), 4.5)
