"""CPU oracle for the PITCH KV-cache codec: a numpy restatement of the reference specification.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or as the timed CPU baseline). The product
path (``pitch_amd``) never imports it; the product runs on the HIP library or raises.

Every function restates the arithmetic of ``reference/pitch_reference.py`` (cited per function): float64
rotation, float32 codebook midpoints, ``searchsorted(side="left")``, float32 KIVI arithmetic and
round-to-nearest-even fp16 ranges. The operation order is kept where it decides rounding (division by the
norm before the sign flip, division by sqrt(d) after the transform, ``/ step + 0.5`` in float32).
``pack_codes``/``unpack_codes`` are vectorised over the word layout instead of the reference's per-column
Python loop; the bit layout is the same (checked against the fixtures and a brute-force packer in tests).

Pinning (tests/test_oracle_*.py): every function is checked against the reference's golden vectors
(tests/golden/parity.json, channel_parity.json), against vectors written from the reference at the
shapes those fixtures do not cover (tests/golden/ref_vectors.npz), and against closed forms
(Sylvester Hadamard matrix via scipy, H.H = d.I, one-hot error 0.25, zero vector, PCG hash from
Python integers, brute-force bit packing).
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

DEFAULT_SEED = 0x50495443          # reference/pitch_reference.py:7 (PITCH.defaultSeed, "PITC")
SUPPORTED_BITS = range(2, 9)       # reference/pitch_reference.py:8
SUPPORTED_DIMS = [2 ** k for k in range(1, 11)]   # reference/pitch_reference.py:9
CHANNEL_DEFAULT_GROUP = 64         # reference/pitch_reference.py:137
FP16_MAX = 65504.0                 # reference/pitch_reference.py:138

_CODEBOOK_PATH = Path(__file__).resolve().parent.parent / "pitch_amd" / "data" / "codebooks.json"
_codebooks: dict | None = None


# ----------------------------------------------------------------------------- rotation
def pcg_hash(v):
    """32-bit PCG-RXS-M-XS hash. Follows reference/pitch_reference.py:11-15 (and PITCHKernels.metal:26-31)."""
    v = np.asarray(v, dtype=np.uint64)
    state = (v * np.uint64(747796405) + np.uint64(2891336453)) & np.uint64(0xFFFFFFFF)
    word = (((state >> ((state >> np.uint64(28)) + np.uint64(4))) ^ state) * np.uint64(277803737)) \
        & np.uint64(0xFFFFFFFF)
    return ((word >> np.uint64(22)) ^ word) & np.uint64(0xFFFFFFFF)


def rand_signs(seed: int, d: int) -> np.ndarray:
    """+1.0 where pcg_hash(seed + i mod 2^32) is odd, else -1.0. reference/pitch_reference.py:17-19."""
    h = pcg_hash((np.uint64(seed) + np.arange(d, dtype=np.uint64)) & np.uint64(0xFFFFFFFF))
    return np.where(h & np.uint64(1), 1.0, -1.0)


def wht(x: np.ndarray) -> np.ndarray:
    """Unnormalised natural-order (Sylvester) fast Walsh-Hadamard transform over rows, float64.

    Stage h = 1, 2, 4, ...: (a, b) -> (a + b, a - b) for the pair (i, i + h) with bit h of i clear.
    reference/pitch_reference.py:21-31.
    """
    x = np.array(x, dtype=np.float64, copy=True)
    n, d = x.shape
    h = 1
    while h < d:
        v = x.reshape(n, d // (2 * h), 2, h)
        a = v[:, :, 0, :].copy()
        b = v[:, :, 1, :].copy()
        v[:, :, 0, :] = a + b
        v[:, :, 1, :] = a - b
        h *= 2
    return x


def rotate(X, seed):
    """y = H (s * x) / sqrt(d). reference/pitch_reference.py:33."""
    return wht(X * rand_signs(seed, X.shape[1])) / math.sqrt(X.shape[1])


def unrotate(Y, seed):
    """x = s * (H y) / sqrt(d). reference/pitch_reference.py:34."""
    return wht(Y) * rand_signs(seed, Y.shape[1]) / math.sqrt(Y.shape[1])


# ----------------------------------------------------------------------------- codebooks
def turbo_codebook(d: int, b: int) -> np.ndarray:
    """Lloyd-Max table (d, b) from codebooks.json, read as float32 then widened. pitch_reference.py:56-63."""
    global _codebooks
    if _codebooks is None:
        _codebooks = json.loads(_CODEBOOK_PATH.read_text())
    return np.array(_codebooks[f"{d}_{b}"], dtype=np.float32).astype(np.float64)


def turbo_edges(d: int, b: int) -> np.ndarray:
    """Decision boundaries float32(0.5f * (c[k] + c[k+1])) widened to float64. pitch_reference.py:99-100."""
    cb32 = turbo_codebook(d, b).astype(np.float32)
    return (np.float32(0.5) * (cb32[1:] + cb32[:-1])).astype(np.float64)


def code_stride_bytes(d: int, b: int) -> int:
    """Bytes of packed codes per vector, a whole number of 32-bit words. pitch_reference.py:65-66."""
    return ((d * b + 7) // 8 + 3) & ~3


# ----------------------------------------------------------------------------- packing
def pack_codes(codes: np.ndarray, b: int) -> bytes:
    """Code i occupies bits [i*b, i*b + b) of the vector's little-endian uint32 word stream.

    Same layout as reference/pitch_reference.py:68-78; built from a 64-bit window per word instead of a
    per-column loop.
    """
    codes = np.asarray(codes)
    n, d = codes.shape
    words = code_stride_bytes(d, b) // 4
    out = np.zeros((n, words), dtype=np.uint64)
    c = codes.astype(np.uint64) & np.uint64((1 << b) - 1)
    for i in range(d):
        start = i * b
        w, off = start >> 5, start & 31
        out[:, w] |= (c[:, i] << np.uint64(off)) & np.uint64(0xFFFFFFFF)
        if off + b > 32:
            out[:, w + 1] |= c[:, i] >> np.uint64(32 - off)
    return out.astype("<u4").tobytes()


def unpack_codes(buf: bytes, n: int, d: int, b: int) -> np.ndarray:
    """Inverse of pack_codes. reference/pitch_reference.py:80-90."""
    words = np.frombuffer(bytes(buf), dtype="<u4").astype(np.uint64).reshape(n, -1)
    codes = np.zeros((n, d), dtype=np.int64)
    mask = np.uint64((1 << b) - 1)
    for i in range(d):
        start = i * b
        w, off = start >> 5, start & 31
        v = words[:, w] >> np.uint64(off)
        if off + b > 32:
            v |= words[:, w + 1] << np.uint64(32 - off)
        codes[:, i] = (v & mask).astype(np.int64)
    return codes


# ----------------------------------------------------------------------------- per-vector codecs
def turbo_encode(X: np.ndarray, b: int, seed: int = DEFAULT_SEED):
    """(codes (n, d) int64, norms (n,) float64). reference/pitch_reference.py:92-102."""
    X = np.asarray(X, dtype=np.float64)
    d = X.shape[1]
    norms = np.linalg.norm(X, axis=1)
    safe = np.where(norms > 0, norms, 1.0)[:, None]
    U = rotate(X / safe, seed)
    codes = np.searchsorted(turbo_edges(d, b), U, side="left")
    return codes, norms


def turbo_rotated(X: np.ndarray, seed: int = DEFAULT_SEED) -> np.ndarray:
    """The float64 rotated unit vectors U that turbo_encode quantises (for boundary classification)."""
    X = np.asarray(X, dtype=np.float64)
    norms = np.linalg.norm(X, axis=1)
    safe = np.where(norms > 0, norms, 1.0)[:, None]
    return rotate(X / safe, seed)


def turbo_decode(codes: np.ndarray, norms: np.ndarray, b: int, seed: int = DEFAULT_SEED):
    """x = unrotate(c[codes]) * norm, float64. reference/pitch_reference.py:104-107."""
    d = codes.shape[1]
    U = turbo_codebook(d, b)[codes]
    return unrotate(U, seed) * np.asarray(norms, dtype=np.float64)[:, None]


def polar_parts(X: np.ndarray, seed: int = DEFAULT_SEED):
    """(r, theta in [0, 2pi)) per coordinate pair of rotate(x). reference/pitch_reference.py:110-113."""
    Y = rotate(np.asarray(X, dtype=np.float64), seed)
    a, c = Y[:, 0::2], Y[:, 1::2]
    return np.hypot(a, c), np.mod(np.arctan2(c, a), 2 * np.pi)


def polar_encode(X: np.ndarray, b: int, seed: int = DEFAULT_SEED):
    """Even code = radius on [0, rmax] in 2^b - 1 steps, odd code = angle in 2^b circular bins.

    Returns (codes (n, d) int64, rmax (n,) float64). reference/pitch_reference.py:109-121.
    """
    r, theta = polar_parts(X, seed)
    RL = 2 ** b - 1
    N = 2 ** b
    rmax = r.max(axis=1)
    safe = np.where(rmax > 0, rmax, 1.0)[:, None]
    rq = np.clip(np.floor(r / safe * RL + 0.5), 0, RL)
    tq = np.mod(np.floor(theta / (2 * np.pi) * N + 0.5), N)
    codes = np.empty((r.shape[0], 2 * r.shape[1]), dtype=np.int64)
    codes[:, 0::2] = rq
    codes[:, 1::2] = tq
    return codes, rmax


def polar_decode(codes: np.ndarray, rmax: np.ndarray, b: int, seed: int = DEFAULT_SEED):
    """(r cos t, r sin t) interleaved, then unrotate. reference/pitch_reference.py:123-129."""
    RL = 2 ** b - 1
    N = 2 ** b
    r = codes[:, 0::2] / RL * np.asarray(rmax, dtype=np.float64)[:, None]
    theta = codes[:, 1::2] / N * 2 * np.pi
    Y = np.empty(codes.shape)
    Y[:, 0::2] = r * np.cos(theta)
    Y[:, 1::2] = r * np.sin(theta)
    return unrotate(Y, seed)


ENCODERS = {"turboQuant": turbo_encode, "polarQuant": polar_encode}   # pitch_reference.py:131
DECODERS = {"turboQuant": turbo_decode, "polarQuant": polar_decode}   # pitch_reference.py:132


def bits_per_coordinate(d: int, b: int) -> float:
    """(codeStride + 4-byte scale) * 8 / d. reference/pitch_reference.py:134-135."""
    return (code_stride_bytes(d, b) + 4) * 8 / d


# ----------------------------------------------------------------------------- per-channel (KIVI) keys
def channel_group_count(n: int, G: int) -> int:
    """reference/pitch_reference.py:141-142."""
    return (n + G - 1) // G


def channel_encode(X: np.ndarray, b: int, G: int = CHANNEL_DEFAULT_GROUP):
    """Per group of G tokens and per channel: fp16 (min, max), then uniform b-bit codes, all float32.

    Returns (codes (n, d) int64, ranges (groups, 2, d) float16). reference/pitch_reference.py:145-162.
    """
    X = np.asarray(X, dtype=np.float32)
    n, d = X.shape
    if not np.isfinite(X).all() or np.abs(X).max() > FP16_MAX:
        raise ValueError("inputs must be finite with magnitude at most 65504 (fp16 range)")
    L = np.float32(2 ** b - 1)
    codes = np.empty((n, d), dtype=np.int64)
    ranges = np.empty((channel_group_count(n, G), 2, d), dtype=np.float16)
    for g, s in enumerate(range(0, n, G)):
        blk = X[s:s + G]
        lo16, hi16 = blk.min(0).astype(np.float16), blk.max(0).astype(np.float16)
        lo = lo16.astype(np.float32)
        step = (hi16.astype(np.float32) - lo) / L
        step[step == 0] = np.float32(1)
        q = np.floor((blk - lo) / step + np.float32(0.5))
        codes[s:s + G] = np.clip(q, 0, L).astype(np.int64)
        ranges[g, 0], ranges[g, 1] = lo16, hi16
    return codes, ranges


def channel_decode(codes: np.ndarray, ranges: np.ndarray, b: int, G: int = CHANNEL_DEFAULT_GROUP):
    """x = f32(code) * step + lo, float32 with no fused multiply-add. reference/pitch_reference.py:165-174."""
    n, d = codes.shape
    L = np.float32(2 ** b - 1)
    out = np.empty((n, d), dtype=np.float32)
    for g, s in enumerate(range(0, n, G)):
        lo = ranges[g, 0].astype(np.float32)
        step = (ranges[g, 1].astype(np.float32) - lo) / L
        step[step == 0] = np.float32(1)
        out[s:s + G] = codes[s:s + G].astype(np.float32) * step + lo
    return out


def channel_bits_per_coordinate(d: int, b: int, G: int = CHANNEL_DEFAULT_GROUP) -> float:
    """reference/pitch_reference.py:177-178."""
    return code_stride_bytes(d, b) * 8 / d + 32 / G


# ----------------------------------------------------------------------------- 16-bit element types
# The reference reads and writes float32 only and leaves float16 / bfloat16 caches to a conversion by the
# caller ("Inputs and outputs are float32; models that keep caches in fp16 or bf16 need a conversion",
# README.md:97). The 16-bit entry points are specified as exactly that conversion: a 16-bit input is widened
# to float32 (exact for both types) and encoded as float32; a 16-bit output is the float32 decode rounded to
# nearest even. These helpers state the two roundings; tests/test_io_rounding.py pins them against torch's
# and numpy's own conversions.
IO_TYPES = ("float32", "float16", "bfloat16")


def bf16_bits(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even; NaN -> quiet NaN of the same sign, and a
    finite value beyond the largest bfloat16 rounds to infinity."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))) >> np.uint64(16))
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    quiet = (u >> np.uint64(16)) | np.uint64(0x40)
    return np.where(nan, quiet, rounded).astype(np.uint16)


def bf16_to_f32(bits) -> np.ndarray:
    """bfloat16 bit patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def to_io_bits(x, io: str) -> np.ndarray:
    """float32 values -> the element type's bit patterns (float32 bits unchanged; 16-bit types RNE)."""
    x = np.asarray(x, dtype=np.float32)
    if io == "float32":
        return x.view(np.uint32)
    if io == "float16":
        with np.errstate(over="ignore"):                      # beyond 65504 rounds to infinity
            return x.astype(np.float16).view(np.uint16)
    if io == "bfloat16":
        return bf16_bits(x)
    raise ValueError(io)


def from_io_bits(bits, io: str) -> np.ndarray:
    """The element type's bit patterns -> float32 (exact)."""
    if io == "float32":
        return np.asarray(bits, dtype=np.uint32).view(np.float32)
    if io == "float16":
        return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)
    if io == "bfloat16":
        return bf16_to_f32(bits)
    raise ValueError(io)


def round_io(x, io: str) -> np.ndarray:
    """float32 values rounded to the element type and widened back (what a 16-bit decode holds)."""
    return from_io_bits(to_io_bits(x, io), io)


# ----------------------------------------------------------------------------- key-bias removal
def rotate_half(x: np.ndarray) -> np.ndarray:
    """(-x[d/2:], x[:d/2]) along the last axis: the rotate_half of the RoPE models the reference evaluates
    (reference/mechanism_eval.py:84, the model module's own rotate_half)."""
    d = x.shape[-1]
    return np.concatenate([-x[..., d // 2:], x[..., :d // 2]], axis=-1)


def key_bias_offsets(bias, cos, sin, first_position: int, count: int, heads: int) -> np.ndarray:
    """R_t b_h for vectors 0..count-1 of a token-major [t][h] cache: token first_position + v // heads, head
    v % heads; bb * cos + rotate_half(bb) * sin in float32 with each product and the sum rounded once
    (reference/mechanism_eval.py:88-97, rotated_bias)."""
    f32 = np.float32
    v = np.arange(count)
    t = first_position + v // heads
    b = np.asarray(bias, f32)[v % heads]
    t1 = (b * np.asarray(cos, f32)[t]).astype(f32)
    t2 = (rotate_half(b) * np.asarray(sin, f32)[t]).astype(f32)
    return (t1 + t2).astype(f32)


# ----------------------------------------------------------------------------- attention on decoded caches
def log_softmax(S: np.ndarray) -> np.ndarray:
    """Row-wise log-softmax, float64. reference/attention_eval.py:31-33."""
    m = S.max(axis=-1, keepdims=True)
    return S - m - np.log(np.exp(S - m).sum(axis=-1, keepdims=True))


def attend(Q: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float):
    """Attention of queries Q (m, d) over keys K (T, d) and values V (T, d), float64: S = Q K^T * scale,
    log-softmax, exp(lp) V. reference/attention_extra.py:70-74 without the causal mask, since a decode-step query
    sees every cached token. Returns (O (m, d), lse (m,)) with lse = log sum_t exp(S_t)."""
    S = (np.asarray(Q, np.float64) @ np.asarray(K, np.float64).T) * scale
    lp = log_softmax(S)
    m = S.max(axis=-1)
    lse = m + np.log(np.exp(S - m[:, None]).sum(axis=-1))
    return np.exp(lp) @ np.asarray(V, np.float64), lse


def attention_decode(Q, k_codes, k_scales, v_codes, v_scales, k_method: str, k_bits: int, v_method: str,
                     v_bits: int, scale: float, k_seed: int = DEFAULT_SEED, v_seed: int = DEFAULT_SEED):
    """Attention over the decodes of compressed caches, the way the reference evaluates it
    (reference/attention_extra.py:11-14 decodes with pitch_reference, then attend): K = decode(k_codes, k_scales),
    V = decode(v_codes, v_scales), with float32 scales widened (attention_extra.py:13). Q (m, d); codes (T, d)."""
    K = DECODERS[k_method](k_codes, np.asarray(k_scales, np.float32).astype(np.float64), k_bits, k_seed)
    V = DECODERS[v_method](v_codes, np.asarray(v_scales, np.float32).astype(np.float64), v_bits, v_seed)
    return attend(Q, K, V, scale)


def attention_decode_channel_keys(Q, k_codes, k_ranges, k_bits: int, G: int, v_codes, v_scales, v_method: str,
                                  v_bits: int, scale: float, v_seed: int = DEFAULT_SEED):
    """Attention with per-channel keys and per-vector values ("kivi_K{b}_turboV{b}",
    reference/attention_extra.py:57-59): K = channel_decode(k_codes, k_ranges) in float32
    (pitch_reference.py:165-174), V = decode(v_codes, v_scales), then attend."""
    K = channel_decode(k_codes, k_ranges, k_bits, G)
    V = DECODERS[v_method](v_codes, np.asarray(v_scales, np.float32).astype(np.float64), v_bits, v_seed)
    return attend(Q, K, V, scale)


# ----------------------------------------------------------------------------- boundary classification
# The parity bar for per-vector codes: a code may differ from the oracle's only at a coordinate whose
# rotated value lies within REL_BAND of a decision boundary, relative to max(|boundary|, floor). The floor
# handles the exactly-zero middle edge: it is 1/sqrt(d) (the typical |u| of a unit vector's coordinate)
# for TurboQuant, and 1 for the rounding points of the polar and KIVI quantisers, whose argument is
# already on the code scale.
REL_BAND = 1e-6


def turbo_near_boundary(U: np.ndarray, b: int, rel: float = REL_BAND) -> np.ndarray:
    """Mask of coordinates of U (n, d) within rel of a TurboQuant decision edge."""
    d = U.shape[1]
    edges = turbo_edges(d, b)
    idx = np.searchsorted(edges, U, side="left")
    lo = edges[np.clip(idx - 1, 0, len(edges) - 1)]
    hi = edges[np.clip(idx, 0, len(edges) - 1)]
    dist = np.minimum(np.abs(U - lo), np.abs(U - hi))
    scale = np.maximum(np.minimum(np.abs(lo), np.abs(hi)), 1.0 / math.sqrt(d))
    return dist <= rel * scale


def _near_integer(t: np.ndarray, rel: float) -> np.ndarray:
    """Within rel * max(|t|, 1) of a rounding point: floor(t) is decided by an integer boundary."""
    return np.abs(t - np.round(t)) <= rel * np.maximum(np.abs(t), 1.0)


def polar_near_boundary(X: np.ndarray, b: int, seed: int = DEFAULT_SEED, rel: float = REL_BAND) -> np.ndarray:
    """Mask (n, d) of polar codes whose rounding argument lies within rel of a rounding point."""
    r, theta = polar_parts(X, seed)
    RL, N = 2 ** b - 1, 2 ** b
    rmax = r.max(axis=1)
    safe = np.where(rmax > 0, rmax, 1.0)[:, None]
    tr = r / safe * RL + 0.5
    ta = theta / (2 * np.pi) * N + 0.5
    mask = np.zeros((r.shape[0], 2 * r.shape[1]), dtype=bool)
    mask[:, 0::2] = _near_integer(tr, rel)
    # a pair at the origin decides its angle by the signs of its zeros, so it counts as on a boundary
    mask[:, 1::2] = _near_integer(ta, rel) | (r == 0)
    return mask


def channel_near_boundary(X: np.ndarray, b: int, G: int = CHANNEL_DEFAULT_GROUP,
                          rel: float = REL_BAND) -> np.ndarray:
    """Mask (n, d) of KIVI codes whose float32 (x - lo) / step + 0.5 lies within rel of an integer."""
    X = np.asarray(X, dtype=np.float32)
    n, d = X.shape
    L = np.float32(2 ** b - 1)
    out = np.zeros((n, d), dtype=bool)
    for s in range(0, n, G):
        blk = X[s:s + G]
        lo16, hi16 = blk.min(0).astype(np.float16), blk.max(0).astype(np.float16)
        lo = lo16.astype(np.float32)
        step = (hi16.astype(np.float32) - lo) / L
        step[step == 0] = np.float32(1)
        t = ((blk - lo) / step + np.float32(0.5)).astype(np.float64)
        out[s:s + G] = _near_integer(t, rel)
    return out
