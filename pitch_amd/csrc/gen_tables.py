#!/usr/bin/env python3
"""Generates pitch_tables.inc: the constant tables the HIP kernels read.

* The 70 Lloyd-Max codebooks of pitch_amd/data/codebooks.json as float32, keyed by (dim, bits) like the
  reference's generated table (Sources/PITCH/TurboCodebooks.swift:10-84).
* Their decision edges float32(0.5f * (c[k] + c[k+1])), computed in float32 exactly as
  reference/pitch_reference.py:99-100 does, so the encoder compares against the same values.
* For PolarQuant decode (reference/pitch_reference.py:123-129): per bit width, the radius fractions
  k / (2^b - 1) and the unit vectors (cos, sin)(k / 2^b * 2 * pi), evaluated in float64 with the
  reference's operation order and rounded once to float32.
* The bucket tables of the TurboQuant encoder (lut_for) and the float32 atan polynomials of the PolarQuant
  encoder's fast angle path (atan_poly), each checked here against the exact answer.
* For the PolarQuant encoder's angle codes at b <= 5: the tangents of the sector boundaries inside the first
  octant, RN(tan((k - 1/2) 2 pi / 2^b)) for k = 1 .. ceil(2^b / 8) (sector_tans).

Usage: python gen_tables.py <codebooks.json> <out.inc>
"""
from __future__ import annotations

import json
import sys

import numpy as np

DIMS = [2 ** k for k in range(1, 11)]
BITS = range(2, 9)


def _floats(vals) -> str:
    """Exact C++ hex-float literals of float32 values (+inf as a builtin)."""
    return ",".join("__builtin_inff()" if np.isinf(v) else float(np.float32(v)).hex() + "f" for v in vals)


MAX_LUT = 2048      # entries per bucket table (8 bytes each); larger tables fall back to binary search
GUARD = 1e-6        # minimum distance, in bucket units, between any edge and any bucket boundary


def lut_for(edges: np.ndarray, b: int, full: bool = True):
    """Bucket table for code = #{edges < u} (searchsorted 'left', reference/pitch_reference.py:99-101).

    Buckets have width 2^-m and are indexed by j = floor(u * 2^m + off), clamped to [0, n); off = K + 0.5 puts
    the exactly-zero middle edge inside a bucket; with full=True, K > 2^m + 1 makes every |u| <= 1 land inside
    the table, so only the upper clamp is needed. m is chosen so each bucket holds at most one edge and no
    edge lies within GUARD (in bucket units) of a bucket boundary, which makes an index that is off by one
    (from rounding u * 2^m + off near a boundary) harmless. Then code = c_j + [u > e_j] with
    c_j = #{edges < lower end of bucket j} and e_j = edges[c_j] (+inf past the last edge).
    Returns (2^m, off, [(float32 bits of e_j, c_j)]) or None when the table would exceed MAX_LUT entries.
    """
    L = 2 ** b
    gap = float(np.min(np.diff(edges)))
    m = int(np.ceil(np.log2(2.0 / gap)))
    while True:
        scale = 2.0 ** m
        K = int(np.ceil(float(np.max(np.abs(edges))) * scale)) + 1
        if full:  # cover |u| <= 1 (a coordinate of a rotated unit vector): the index needs no lower clamp
            K = max(K, int(scale) + 2)
        n = 2 * K + 1
        if n > MAX_LUT:
            return None
        off = K + 0.5
        t = edges * scale + off
        frac = np.abs(t - np.round(t))
        counts = np.bincount(np.floor(t).astype(np.int64), minlength=n)
        if frac.min() >= GUARD and counts.max() <= 1:
            break
        m += 1
    lo = (np.arange(n) - off) / scale                  # exact: off and scale are exact, n < 2^20
    c = np.searchsorted(edges, lo, side="left")       # number of edges strictly below the lower end
    ent = []
    for j in range(n):
        e = np.float32(edges[c[j]]) if c[j] < L - 1 else np.float32(np.inf)
        ent.append((int(e.view(np.uint32)), int(c[j])))
    # brute-force check against searchsorted on random points and on points next to every boundary
    rng = np.random.default_rng(b)
    u = np.concatenate([rng.uniform(-1.1, 1.1, 20000), edges, np.nextafter(edges, 2), np.nextafter(edges, -2),
                        lo, np.nextafter(lo, 2), np.nextafter(lo, -2), [0.0, -0.0, 1.0, -1.0]])
    j = np.clip(np.floor(u * scale + off), 0, n - 1).astype(np.int64)
    e_tab = np.array([np.uint32(e).view(np.float32) for e, _ in ent], dtype=np.float64)
    c_tab = np.array([c for _, c in ent])
    got = c_tab[j] + (u > e_tab[j])
    assert np.array_equal(got, np.searchsorted(edges, u, side="left")), (b, m)
    return scale, off, ent


# atan(z) = z * P(z^2) on [0, 1]: polynomial degree per bit width b, and the float32 error bound (rad) each
# degree must meet. The angle code's t = theta / (2 pi) * 2^b + 0.5 may be off by at most 1e-4 (a third of the
# encoder's guard band); 1e-4 * 2 pi / 2^b less 6e-7 rad for the other float32 roundings is the budget.
ATAN_DEG = {2: 4, 3: 4, 4: 5, 5: 5, 6: 6, 7: 6, 8: 7}
ATAN_MAX_ERR = {4: 4e-5, 5: 6e-6, 6: 1e-6, 7: 2e-7}


def atan_eval32(c32, zt):
    """z * P(z^2) in float32 with fused multiply-adds, as the encoder evaluates it."""
    zt = np.asarray(zt, np.float32)
    st = (zt * zt).astype(np.float32)
    p = np.full_like(st, c32[-1])
    for c in c32[-2::-1]:
        p = (p.astype(np.float64) * st + np.float64(c)).astype(np.float32)
    return (p.astype(np.float64) * zt).astype(np.float32)


def atan_poly(deg: int = 7):
    """Least-squares fit of atan(z) / z as a polynomial of degree deg in s = z^2 over [0, 1] (Chebyshev-spaced
    and uniform nodes), rounded to float32. The PolarQuant encoder evaluates z * P(z^2) in float32 for its fast
    angle path; the float32 evaluation error is checked here on a dense grid against ATAN_MAX_ERR[deg]."""
    z = np.concatenate([np.cos(np.linspace(0, np.pi / 2, 20001)), np.linspace(0, 1, 20001)])
    s = z * z
    f = np.where(z > 0, np.arctan(z) / np.where(z > 0, z, 1), 1.0)
    coef, *_ = np.linalg.lstsq(np.vander(s, deg + 1, increasing=True), f, rcond=None)
    c32 = coef.astype(np.float32)
    zt = np.linspace(0, 1, 1000001).astype(np.float32)
    err = np.abs(atan_eval32(c32, zt).astype(np.float64) - np.arctan(zt.astype(np.float64))).max()
    assert err < ATAN_MAX_ERR[deg], (deg, err)
    return c32


SECTOR_BITS = range(2, 6)  # bit widths whose angle codes the encoder decides by boundary comparisons


def sector_tans(b: int) -> np.ndarray:
    """float32 tangents of the angle-code boundaries (k - 1/2) * 2 pi / 2^b inside the first octant [0, pi / 4]
    (pitch_reference.py:117 rounds theta / (2 pi) * 2^b + 0.5 down, so code k starts half a sector below k).
    At b = 2 the only boundary is the octant's edge, pi / 4, whose tangent is 1."""
    k = np.arange(1, ((1 << b) + 7) // 8 + 1, dtype=np.float64)
    t = np.tan((k - 0.5) * 2 * np.pi / (1 << b)).astype(np.float32)
    assert np.all(t <= 1) and np.all(np.diff(t) > 0)
    return t


def main(src: str, dst: str) -> None:
    books = json.loads(open(src).read())
    cb_all, edge_all = [], []
    lines = ["// Generated by pitch_amd/csrc/gen_tables.py from codebooks.json. Do not edit.", ""]
    offs = {}
    for d in DIMS:
        for b in BITS:
            cb = np.array(books[f"{d}_{b}"], dtype=np.float32)
            assert cb.shape == (2 ** b,) and np.all(np.diff(cb) > 0), (d, b)
            edges = (np.float32(0.5) * (cb[1:] + cb[:-1])).astype(np.float32)
            offs[(d, b)] = len(cb_all)
            cb_all.extend(cb.tolist())
            edge_all.extend(edges.tolist() + [float("inf")])     # padded to 2^b with +inf
    lines.append(f"static __device__ const float pitch_codebook_tab[{len(cb_all)}] = {{{_floats(cb_all)}}};")
    lines.append(f"static __device__ const float pitch_edge_tab[{len(edge_all)}] = {{{_floats(edge_all)}}};")
    # table (d, b) starts at (log2 d - 1) * 508 + 2^b - 4 in both arrays (508 = sum of 2^b over b = 2..8)
    for (d, b), off in offs.items():
        assert off == (d.bit_length() - 2) * 508 + (1 << b) - 4
    lines.append("static constexpr int pitch_codebook_offset(int log2d, int bits) "
                 "{ return (log2d - 1) * 508 + (1 << bits) - 4; }")

    # Bucket tables for TurboQuant encoding (see lut_for): entry j = (float32 bits of the first edge at or
    # above the bucket's lower end, number of edges below the bucket's lower end), read as one 8-byte word.
    lut_words, info = [], []
    for d in DIMS:
        for b in BITS:
            cb = np.array(books[f"{d}_{b}"], dtype=np.float32)
            edges = (np.float32(0.5) * (cb[1:] + cb[:-1])).astype(np.float64)
            lut = lut_for(edges, b, full=False)
            if lut is None:
                info.append("{-1, 0, 0.0, 0.0}")
                continue
            scale, off, ent = lut
            # The TurboQuant encoders compare in the bucket domain t = u * 2^m + off + 2^k + 2^(k-1) (k = 17 -
            # log2 of the table's copies in LDS: 12 ... 17 for 32 ... 1 copies, t in [2^k, 2^(k+1))) and keep each
            # entry's code in the low 8 mantissa bits of its mapped edge: the mapping must be exact and leave those
            # bits zero at every k a kernel can compile.
            for k in range(12, 18):
                magic = 2.0 ** k + 2.0 ** (k - 1) + off
                for e_bits, c in ent:
                    e = float(np.uint32(e_bits).view(np.float32))
                    if np.isinf(e):
                        continue
                    E = np.float64(e * scale + magic)
                    assert float(E) - magic == e * scale and 2.0 ** k <= E < 2.0 ** (k + 1), (d, b, k, e)
                    assert int(E.view(np.uint64)) & 0xFF == 0, (d, b, k, e)
            info.append(f"{{{len(lut_words) // 2}, {len(ent)}, {scale.hex()}, {off.hex()}}}")
            for e_bits, c in ent:
                lut_words.extend([e_bits, c])
    lines.append(f"static __device__ const uint32_t pitch_lut_tab[{len(lut_words)}] = "
                 f"{{{','.join(str(w) for w in lut_words)}}};")
    lines.append("struct PitchLutInfo { int offset; int entries; double scale; double off; };")
    lines.append(f"static constexpr PitchLutInfo pitch_lut_info_tab[{len(info)}] = {{{','.join(info)}}};")
    lines.append("static constexpr PitchLutInfo pitch_lut_info(int log2d, int bits) "
                 "{ return pitch_lut_info_tab[(log2d - 1) * 7 + bits - 2]; }")

    rad, cos_, sin_ = [], [], []
    poffs = {}
    for b in BITS:
        RL, N = 2 ** b - 1, 2 ** b
        k = np.arange(N, dtype=np.float64)
        poffs[b] = len(rad)
        rad.extend((k / RL).astype(np.float32).tolist())
        theta = k / N * 2 * np.pi
        cos_.extend(np.cos(theta).astype(np.float32).tolist())
        sin_.extend(np.sin(theta).astype(np.float32).tolist())
    lines.append(f"static __device__ const float pitch_polar_radius_tab[{len(rad)}] = {{{_floats(rad)}}};")
    lines.append(f"static __device__ const float pitch_polar_cos_tab[{len(cos_)}] = {{{_floats(cos_)}}};")
    lines.append(f"static __device__ const float pitch_polar_sin_tab[{len(sin_)}] = {{{_floats(sin_)}}};")
    lines.append("static constexpr int pitch_polar_offset(int bits) { return (1 << bits) - 4; }")
    # fitted atan polynomials: row deg holds the deg + 1 coefficients of degree deg (zero-padded)
    rows = []
    for deg in range(9):
        c = atan_poly(deg) if deg in ATAN_MAX_ERR else np.zeros(0, np.float32)
        rows.append("{" + _floats(list(c) + [0.0] * (9 - len(c))) + "}")
    lines.append(f"static constexpr float pitch_atan_coef[9][9] = {{{','.join(rows)}}};")
    lines.append("static constexpr int pitch_atan_degree(int bits) { return "
                 + " : ".join(f"bits == {b} ? {d}" for b, d in ATAN_DEG.items()) + " : 7; }")
    # sector-boundary tangents: row b - 2 holds the ceil(2^b / 8) tangents of bit width b (zero-padded)
    rows = ["{" + _floats(list(sector_tans(b)) + [0.0] * (4 - len(sector_tans(b)))) + "}" for b in SECTOR_BITS]
    lines.append(f"static constexpr float pitch_sector_tan[{len(rows)}][4] = {{{','.join(rows)}}};")
    for b in BITS:
        assert poffs[b] == (1 << b) - 4
    open(dst, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    main(sys.argv[1], sys.argv[2])
