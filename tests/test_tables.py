"""The constant tables the HIP kernels read, checked on the CPU against the oracle (CPU only).

pitch_amd/csrc/gen_tables.py writes the codebooks, the float32 decision edges, the PolarQuant decode tables
and the bucket tables of the TurboQuant encoder. The bucket quantiser replaces the reference's boundary
search (searchsorted 'left', reference/pitch_reference.py:99-101) with code = c_j + [u > e_j] for
j = clamp(floor(u * 2^m + off)); here it is evaluated in numpy exactly as the kernel does (float64 u, float32
edge widened) on random points and on the float64 neighbours of every edge and bucket boundary.
"""
import importlib.util
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import pitch_oracle as O

ROOT = Path(__file__).resolve().parent.parent
_spec = importlib.util.spec_from_file_location("gen_tables", ROOT / "pitch_amd" / "csrc" / "gen_tables.py")
G = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(G)


@pytest.mark.parametrize("d", O.SUPPORTED_DIMS)
def test_bucket_quantiser_equals_boundary_search(d):
    rng = np.random.default_rng(d)
    for b in O.SUPPORTED_BITS:
        edges = O.turbo_edges(d, b)
        lut = G.lut_for(edges, b, full=False)
        if lut is None:                  # the kernel falls back to a binary search over the edges
            continue
        scale, off, ent = lut
        n = len(ent)
        assert n <= G.MAX_LUT
        e_tab = np.array([np.uint32(e).view(np.float32) for e, _ in ent], dtype=np.float64)
        c_tab = np.array([c for _, c in ent])
        lo = (np.arange(n) - off) / scale
        u = np.concatenate([rng.uniform(-1, 1, 100000) * (1.2 if d < 16 else 4 / np.sqrt(d)),
                            *[np.nextafter(edges, s) for s in (2, -2)], edges,
                            *[np.nextafter(lo, s) for s in (2, -2)], lo, [0.0, -0.0, 1.0, -1.0, 1e-300]])
        j = np.clip(np.floor(np.maximum(u * scale + off, 0.0)), 0, n - 1).astype(np.int64)
        got = c_tab[j] + (u > e_tab[j])
        assert np.array_equal(got, np.searchsorted(edges, u, side="left")), (d, b)


def test_generated_include(tmp_path):
    out = tmp_path / "t.inc"
    G.main(str(ROOT / "pitch_amd" / "data" / "codebooks.json"), str(out))
    text = out.read_text()
    for name in ("pitch_codebook_tab", "pitch_edge_tab", "pitch_lut_tab", "pitch_polar_radius_tab",
                 "pitch_polar_cos_tab", "pitch_polar_sin_tab"):
        assert name in text


def test_codebook_data_matches_oracle_tables():
    books = json.loads((ROOT / "pitch_amd" / "data" / "codebooks.json").read_text())
    assert len(books) == 70
    for d in O.SUPPORTED_DIMS:
        for b in O.SUPPORTED_BITS:
            assert np.array_equal(np.array(books[f"{d}_{b}"], np.float32).astype(np.float64), O.turbo_codebook(d, b))
