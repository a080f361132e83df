"""Loaders for the golden vectors under tests/golden (reference fixtures and vectors written from the
reference by tests/golden/gen_ref_vectors.py). Data only; decoding follows reference/gen_fixtures.py:21-22."""
from __future__ import annotations

import base64
import functools
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"


def f32(s: str) -> np.ndarray:
    return np.frombuffer(base64.b64decode(s), dtype="<f4")


def u16(s: str) -> np.ndarray:
    return np.frombuffer(base64.b64decode(s), dtype="<u2")


@functools.lru_cache(maxsize=None)
def parity():
    """(groups {name: (n, d) float32}, cases [dict]) of parity.json (40 per-vector cases)."""
    p = json.loads((GOLDEN / "parity.json").read_text())
    groups = {g["name"]: f32(g["input"]).reshape(g["count"], g["dim"]) for g in p["groups"]}
    return groups, p["cases"]


@functools.lru_cache(maxsize=None)
def channel_parity():
    """(groups, cases) of channel_parity.json (17 per-channel cases)."""
    p = json.loads((GOLDEN / "channel_parity.json").read_text())
    groups = {g["name"]: f32(g["input"]).reshape(g["count"], g["dim"]) for g in p["groups"]}
    return groups, p["cases"]


@functools.lru_cache(maxsize=None)
def ref_vectors():
    z = np.load(GOLDEN / "ref_vectors.npz", allow_pickle=False)
    return {k: z[k] for k in z.files}


def ref_per_vector_cases():
    """[(key, X, method, bits, seed, codes bytes, scales, recon)] from ref_vectors.npz."""
    z = ref_vectors()
    out = []
    for key in z["index"]:
        key = str(key)
        if not key.startswith("pv/"):
            continue
        _, tag, method, b, s = key.split("/")
        out.append((key, z[f"in/{tag}"], method, int(b[1:]), int(s[1:]), z[key + "/codes"].tobytes(),
                    z[key + "/scales"], z[key + "/recon"]))
    return out


def ref_channel_cases():
    """[(key, X, bits, G, codes bytes, ranges uint16, recon)] from ref_vectors.npz."""
    z = ref_vectors()
    out = []
    for key in z["index"]:
        key = str(key)
        if not key.startswith("ch/"):
            continue
        _, tag, b, g = key.split("/")
        out.append((key, z[f"in/{tag}"], int(b[1:]), int(g[1:]), z[key + "/codes"].tobytes(),
                    z[key + "/ranges"], z[key + "/recon"]))
    return out


def config1_inputs() -> np.ndarray:
    """BASELINE config 1 inputs: 4096 x 64 N(0,1) float32 from default_rng(0)."""
    return np.random.default_rng(0).standard_normal((4096, 64)).astype(np.float32)
