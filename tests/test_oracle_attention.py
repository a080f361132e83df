"""The oracle's attention over decoded caches, and the rotated-domain identity the attention kernels use (CPU).

oracle.attend restates reference/attention_extra.py:70-74 (S = Q K^T * scale, log-softmax, P V) for decode-step
queries. It is pinned here against an independent formulation (scipy's softmax and logsumexp) and against closed
forms: identical keys give uniform weights (output = mean of V, lse = s + log T), a dominant key selects its
value, and shifting every score by a constant changes only lse.

The kernels never decode a token: they rotate the query once and read the code tables directly,
q . k_t = n_t / sqrt(d) * (H (s_K (.) q)) . t[c_t] and sum_t p_t v_t = s_V (.) H(sum_t p_t n_t t[c_t]) / sqrt(d).
test_rotated_domain_identity evaluates exactly that algebra in numpy (codebook and polar value tables, pairs of
codes, the workspace's chunked flash-decoding merge in log2 units) and checks it against the oracle, so a
mistake in the derivation (a missing sign, a transposed table, the wrong scale) fails on the CPU.
"""
import math

import numpy as np
import pytest
from scipy.special import logsumexp, softmax

from oracle import pitch_oracle as O


def test_attend_matches_scipy():
    rng = np.random.default_rng(0)
    Q, K, V = rng.standard_normal((5, 64)), rng.standard_normal((300, 64)), rng.standard_normal((300, 64))
    out, lse = O.attend(Q, K, V, 0.125)
    S = Q @ K.T * 0.125
    assert np.allclose(out, softmax(S, axis=1) @ V, rtol=1e-12, atol=1e-12)
    assert np.allclose(lse, logsumexp(S, axis=1), rtol=1e-12, atol=1e-12)


def test_attend_closed_forms():
    rng = np.random.default_rng(1)
    T, d = 37, 16
    V = rng.standard_normal((T, d))
    q = rng.standard_normal((1, d))
    k = rng.standard_normal(d)
    out, lse = O.attend(q, np.tile(k, (T, 1)), V, 0.3)            # identical keys: uniform weights
    assert np.allclose(out[0], V.mean(0), atol=1e-12)
    assert math.isclose(lse[0], 0.3 * float(q[0] @ k) + math.log(T), rel_tol=1e-12)
    K = rng.standard_normal((T, d)) * 1e-3
    K[7] = q[0] * 10                                                # one key dominates
    out, lse = O.attend(q, K, V, 1.0)
    assert np.allclose(out[0], V[7], atol=1e-9)
    # adding alpha * q / |q|^2 to every key adds alpha to every score: same output, lse + alpha
    out2, lse2 = O.attend(q, K + 2.5 * q[0] / float(q[0] @ q[0]), V, 1.0)
    assert np.allclose(out2, out, atol=1e-12) and math.isclose(lse2[0], lse[0] + 2.5, rel_tol=1e-12)


def _tables(method, d, b):
    """Value tables t[c] per coordinate pair as the kernels build them: TurboQuant (cb[c0], cb[c1]); PolarQuant
    (r[c0] cos a[c1], r[c0] sin a[c1]) with r = c0 / (2^b - 1), a = 2 pi c1 / 2^b."""
    L = 2 ** b
    c0, c1 = np.meshgrid(np.arange(L), np.arange(L), indexing="ij")
    if method == "turboQuant":
        cb = O.turbo_codebook(d, b)
        return np.stack([cb[c0], cb[c1]], -1)                       # [c0][c1] -> (x, y)
    r = c0 / (L - 1)
    th = c1 / L * 2 * np.pi
    return np.stack([r * np.cos(th), r * np.sin(th)], -1)


def _rotated_attention(q, kc, ks, vc, vs, k_method, v_method, kb, vb, scale, kseed, vseed, chunk):
    """The kernels' algorithm in float64: rotated query, table reads, chunked softmax in log2 units, merge,
    one inverse rotation."""
    d = q.shape[0]
    Hq = O.wht(q[None] * O.rand_signs(kseed, d))[0]
    qq = Hq * scale * math.log2(math.e) / math.sqrt(d)
    tk, tv = _tables(k_method, d, kb), _tables(v_method, d, vb)
    kval = tk[kc[:, 0::2], kc[:, 1::2]].reshape(len(kc), d)        # rotated-domain key values before the scale
    vval = tv[vc[:, 0::2], vc[:, 1::2]].reshape(len(vc), d)
    s2 = (kval @ qq) * ks                                           # scores in log2 units
    ms, ls, accs = [], [], []
    for c0 in range(0, len(s2), chunk):
        s = s2[c0:c0 + chunk]
        m = s.max()
        p = 2.0 ** (s - m)
        ms.append(m), ls.append(p.sum()), accs.append((p * vs[c0:c0 + chunk]) @ vval[c0:c0 + chunk])
    M = max(ms)
    f = np.array([2.0 ** (m - M) for m in ms])
    lsum = float((np.array(ls) * f).sum())
    a = (np.array(accs) * f[:, None]).sum(0) / lsum
    out = O.rand_signs(vseed, d) * O.wht(a[None])[0] / math.sqrt(d)
    return out, (M + math.log2(lsum)) * math.log(2)


@pytest.mark.parametrize("k_method,v_method,kb,vb", [("turboQuant", "turboQuant", 4, 4), ("polarQuant", "polarQuant", 3, 3),
                                                     ("turboQuant", "polarQuant", 2, 5), ("polarQuant", "turboQuant", 8, 2)])
@pytest.mark.parametrize("d", [64, 128])
def test_rotated_domain_identity(k_method, v_method, kb, vb, d):
    rng = np.random.default_rng(d + kb + 10 * vb)
    T = 700
    kc = rng.integers(0, 2 ** kb, (T, d))
    vc = rng.integers(0, 2 ** vb, (T, d))
    ks = np.exp(rng.uniform(0, 3, T)).astype(np.float32).astype(np.float64)
    vs = np.exp(rng.uniform(-1, 1, T)).astype(np.float32).astype(np.float64)
    q = rng.standard_normal(d)
    ref, ref_lse = O.attention_decode(q[None], kc, ks, vc, vs, k_method, kb, v_method, vb, 1 / math.sqrt(d), 11, 12)
    out, lse = _rotated_attention(q, kc, ks, vc, vs, k_method, v_method, kb, vb, 1 / math.sqrt(d), 11, 12, 256)
    assert np.allclose(out, ref[0], rtol=1e-10, atol=1e-10)
    assert math.isclose(lse, ref_lse[0], rel_tol=1e-10, abs_tol=1e-10)
