"""GPU parity of decode-step attention over compressed caches (pitch_enqueue_attention_decode).

The oracle decodes the caches with the reference's decoders and attends in float64
(oracle.attention_decode: reference/attention_extra.py:11-14, 70-74). The kernels never decode a token; they
read the codes as stored (the algebra is pinned on the CPU by tests/test_oracle_attention.py). Bar, written as
the constants below: per query, the output is within 1e-5 relative L2 of the oracle's and the natural-log
log-sum-exp within 1e-5 (absolute, for |lse| <= 1, else relative). Both are float32 accumulations of O(d)
products per score and O(T) weights per output, whose rounding stays near 1e-6 at these sizes; the scores of
the "peaky" cases reach |s| ~ 40, where a float32 score error of ~1e-6 |s| moves a weight by ~4e-5
relative, so those cases use 1e-4.

Cases cover every kernel instantiation family: d = 64 and 128; key and value bit widths 2..8 (pair tables for
b <= 5, two-level tables above), both methods on either side, different seeds for K and V, query heads per KV
head 1..8 (padded to 1, 2, 4, 8), one to three KV heads, token counts from 1 to 70,000 (one to many chunks,
chunk lengths 256 / 512 / 1024), head-major and token-major caches, and end-to-end encoded caches. Equal key
and value widths run the fused scores-and-values kernel (attn_chunk), including equal widths with different
methods, where it rebuilds its table between the phases; unequal widths run the separate kernels.
"""
import math

import numpy as np
import pytest

from oracle import pitch_oracle as O

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-5
LSE_TOL = 1e-5
PEAKY_TOL = 1e-4


def _rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def _random_cache(rng, kv, T, d, bits, scale_lo, scale_hi):
    codes = rng.integers(0, 2 ** bits, (kv, T, d))
    packed = np.frombuffer(b"".join(O.pack_codes(codes[h], bits) for h in range(kv)), np.uint8).reshape(kv, T, -1)
    scales = np.exp(rng.uniform(scale_lo, scale_hi, (kv, T))).astype(np.float32)
    return codes, packed, scales


def _check(out, lse, ref_out, ref_lse, tol_out, tol_lse, label):
    for i in range(ref_out.shape[0]):
        e = _rel_l2(out[i], ref_out[i])
        assert e < tol_out, f"{label}: query {i} output rel L2 {e}"
    err = np.abs(np.asarray(lse, np.float64) - ref_lse) / np.maximum(1.0, np.abs(ref_lse))
    assert err.max() < tol_lse, f"{label}: lse error {err.max()}"


CASES = [
    # (k_method, v_method, kb, vb, d, nq, kv, T)
    ("turboQuant", "turboQuant", 4, 4, 128, 4, 2, 1000),
    ("turboQuant", "turboQuant", 4, 4, 64, 1, 3, 1000),
    ("turboQuant", "turboQuant", 2, 2, 64, 2, 1, 257),
    ("turboQuant", "turboQuant", 3, 3, 128, 8, 1, 5000),
    ("turboQuant", "turboQuant", 5, 5, 64, 3, 2, 777),
    ("turboQuant", "turboQuant", 6, 6, 128, 5, 1, 300),
    ("turboQuant", "turboQuant", 7, 7, 64, 4, 1, 300),
    ("turboQuant", "turboQuant", 8, 8, 128, 1, 2, 300),
    ("polarQuant", "polarQuant", 4, 4, 128, 4, 2, 1000),
    ("polarQuant", "polarQuant", 2, 2, 64, 6, 1, 256),
    ("polarQuant", "polarQuant", 6, 6, 64, 2, 1, 255),
    ("polarQuant", "polarQuant", 8, 8, 128, 7, 1, 200),
    ("turboQuant", "polarQuant", 4, 3, 128, 4, 1, 600),
    ("turboQuant", "polarQuant", 4, 4, 128, 4, 1, 600),    # equal widths, other tables: the fused kernel rebuilds
    ("polarQuant", "turboQuant", 3, 3, 64, 2, 2, 1300),
    ("polarQuant", "turboQuant", 5, 2, 64, 1, 1, 600),
    ("turboQuant", "turboQuant", 8, 2, 128, 4, 2, 2000),   # the reference's mixed (key, value) bits
    ("turboQuant", "turboQuant", 4, 2, 64, 4, 1, 1),
    ("turboQuant", "turboQuant", 4, 4, 128, 4, 1, 7),
    ("turboQuant", "turboQuant", 4, 4, 128, 4, 2, 70000),  # many chunks, 512-token chunks
    ("turboQuant", "turboQuant", 3, 3, 64, 2, 3, 140000),  # 1024-token chunks
    # unequal widths with 4 or 8 padded query heads: the separate scores and values kernels in matrix-core form
    ("turboQuant", "turboQuant", 4, 2, 64, 8, 2, 3000),
    ("polarQuant", "turboQuant", 3, 4, 128, 7, 1, 1500),
    ("turboQuant", "polarQuant", 2, 3, 64, 3, 2, 900),
]


@pytest.mark.parametrize("k_method,v_method,kb,vb,d,nq,kv,T", CASES)
def test_attention_against_oracle(q, k_method, v_method, kb, vb, d, nq, kv, T):
    import torch
    import pitch_amd as P
    label = f"K {k_method} b{kb} V {v_method} b{vb} d={d} nq={nq} kv={kv} T={T}"
    print(label, flush=True)
    rng = np.random.default_rng(kb * 1000 + vb * 100 + d + nq + kv + T)
    kc, kp, ks = _random_cache(rng, kv, T, d, kb, 1.5, 3.0)
    vc, vp, vs = _random_cache(rng, kv, T, d, vb, -1.0, 1.0)
    Q = rng.standard_normal((kv, nq, d)).astype(np.float32)
    dev = q.device
    kcfg, vcfg = P.QuantConfig(k_method, d, kb, 101), P.QuantConfig(v_method, d, vb, 202)
    out = torch.empty(kv, nq, d, device=dev)
    lse = torch.empty(kv, nq, device=dev)
    q.enqueueAttentionDecode(torch.from_numpy(Q).to(dev), torch.from_numpy(kp.copy()).to(dev),
                             torch.from_numpy(ks).to(dev), torch.from_numpy(vp.copy()).to(dev),
                             torch.from_numpy(vs).to(dev), out, T, kcfg, vcfg, qPerKv=nq, kvHeads=kv, lse=lse)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    for h in range(kv):
        ro, rl = O.attention_decode(Q[h].astype(np.float64), kc[h], ks[h], vc[h], vs[h], k_method, kb, v_method,
                                    vb, 1 / math.sqrt(d), 101, 202)
        _check(out[h], lse[h], ro, rl, OUT_REL_L2, LSE_TOL, f"{label} head {h}")


@pytest.mark.parametrize("d", [64, 128])
def test_attention_peaky_scores(q, d):
    """Sharp softmax: scale 12 / sqrt(d) puts the largest scores near 40."""
    import torch
    import pitch_amd as P
    rng = np.random.default_rng(d)
    T, nq = 3000, 4
    kc, kp, ks = _random_cache(rng, 1, T, d, 4, 1.5, 3.0)
    vc, vp, vs = _random_cache(rng, 1, T, d, 4, -1.0, 1.0)
    Q = rng.standard_normal((1, nq, d)).astype(np.float32)
    cfg = P.QuantConfig("turboQuant", d, 4)
    out = torch.empty(1, nq, d, device=q.device)
    lse = torch.empty(1, nq, device=q.device)
    sc = 12 / math.sqrt(d)
    q.enqueueAttentionDecode(torch.from_numpy(Q).to(q.device), torch.from_numpy(kp.copy()).to(q.device),
                             torch.from_numpy(ks).to(q.device), torch.from_numpy(vp.copy()).to(q.device),
                             torch.from_numpy(vs).to(q.device), out, T, cfg, qPerKv=nq, scale=sc, lse=lse)
    torch.cuda.synchronize()
    ro, rl = O.attention_decode(Q[0].astype(np.float64), kc[0], ks[0], vc[0], vs[0], "turboQuant", 4, "turboQuant",
                                4, sc)
    assert np.abs(rl).max() > 20
    _check(out.cpu().numpy()[0], lse.cpu().numpy()[0], ro, rl, PEAKY_TOL, PEAKY_TOL, f"peaky d={d}")


@pytest.mark.parametrize("method", ["turboQuant", "polarQuant"])
def test_attention_token_major_cache_end_to_end(q, method):
    """Real keys and values, encoded by the library into one token-major [t][h] cache, attended per KV head
    through the strides; compared with the oracle over the library's own codes and with float64 attention over
    the library's float32 decode of the same cache."""
    import torch
    import pitch_amd as P
    dev = q.device
    T, H, d, b, nq = 2000, 4, 128, 4, 2
    g = torch.Generator(device=dev).manual_seed(5)
    K = torch.randn(T, H, d, generator=g, device=dev) * 2 + torch.randn(1, H, d, generator=g, device=dev)
    V = torch.randn(T, H, d, generator=g, device=dev)
    cfg = P.QuantConfig(method, d, b)
    kc = torch.empty(T * H * cfg.codeStride, dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks = torch.empty(T * H, device=dev)
    vs = torch.empty_like(ks)
    q.enqueueEncode(K.contiguous(), kc, ks, T * H, cfg)
    q.enqueueEncode(V.contiguous(), vc, vs, T * H, cfg)
    Q = torch.randn(H, nq, d, generator=g, device=dev)
    out = torch.empty(H, nq, d, device=dev)
    lse = torch.empty(H, nq, device=dev)
    q.enqueueAttentionDecode(Q, kc, ks, vc, vs, out, T, cfg, qPerKv=nq, kvHeads=H, tokenStride=H, headStride=1,
                             lse=lse)
    Kd = torch.empty(T * H, d, device=dev)
    Vd = torch.empty_like(Kd)
    q.enqueueDecode(kc, ks, Kd, T * H, cfg)
    q.enqueueDecode(vc, vs, Vd, T * H, cfg)
    torch.cuda.synchronize()
    codes_k = O.unpack_codes(kc.cpu().numpy().tobytes(), T * H, d, b).reshape(T, H, d)
    codes_v = O.unpack_codes(vc.cpu().numpy().tobytes(), T * H, d, b).reshape(T, H, d)
    ks_np, vs_np = ks.cpu().numpy().reshape(T, H), vs.cpu().numpy().reshape(T, H)
    Kd, Vd = Kd.cpu().numpy().reshape(T, H, d), Vd.cpu().numpy().reshape(T, H, d)
    out, lse, Qn = out.cpu().numpy(), lse.cpu().numpy(), Q.cpu().numpy().astype(np.float64)
    for h in range(H):
        ro, rl = O.attention_decode(Qn[h], codes_k[:, h], ks_np[:, h], codes_v[:, h], vs_np[:, h], method, b, method,
                                    b, 1 / math.sqrt(d))
        _check(out[h], lse[h], ro, rl, OUT_REL_L2, LSE_TOL, f"{method} head {h}")
        ro2, rl2 = O.attend(Qn[h], Kd[:, h], Vd[:, h], 1 / math.sqrt(d))
        _check(out[h], lse[h], ro2, rl2, OUT_REL_L2, LSE_TOL, f"{method} head {h} vs decoded cache")


def test_attention_function_mirror(q):
    import torch
    import pitch_amd as P
    dev = q.device
    rng = np.random.default_rng(3)
    T, d, b = 500, 64, 3
    kc, kp, ks = _random_cache(rng, 2, T, d, b, 1.0, 2.0)
    vc, vp, vs = _random_cache(rng, 2, T, d, b, -1.0, 1.0)
    Q = rng.standard_normal((2, 3, d)).astype(np.float32)
    out, lse = P.attention_decode(torch.from_numpy(Q).to(dev), torch.from_numpy(kp.copy()).to(dev),
                                  torch.from_numpy(ks).to(dev), torch.from_numpy(vp.copy()).to(dev),
                                  torch.from_numpy(vs).to(dev), b)
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    for h in range(2):
        ro, rl = O.attention_decode(Q[h].astype(np.float64), kc[h], ks[h], vc[h], vs[h], "turboQuant", b,
                                    "turboQuant", b, 1 / math.sqrt(d))
        _check(out[h], lse[h], ro, rl, OUT_REL_L2, LSE_TOL, f"mirror head {h}")


CHANNEL_CASES = [
    # (kb, vb, d, G, nq, kv, T)
    (4, 4, 128, 64, 4, 2, 1000),
    (2, 2, 64, 64, 1, 3, 777),
    (3, 4, 128, 128, 6, 1, 5000),
    (8, 2, 64, 64, 4, 2, 300),
    (4, 3, 128, 64, 8, 1, 65),
    (5, 4, 64, 128, 2, 2, 1),
    (4, 4, 128, 64, 4, 1, 70000),
]


@pytest.mark.parametrize("kb,vb,d,G,nq,kv,T", CHANNEL_CASES)
def test_attention_channel_keys(q, kb, vb, d, G, nq, kv, T):
    """Per-channel (KIVI) keys with TurboQuant values: the reference's recommended configuration for biased key
    projections (README.md:30; "kivi_K{b}_turboV{b}", attention_extra.py:57-59). Caches are built by the
    library's own per-head encoders into head-major buffers with the head stride rounded up to the group."""
    import torch
    import pitch_amd as P
    dev = q.device
    label = f"KIVI K b{kb} G{G} / TQ V b{vb} d={d} nq={nq} kv={kv} T={T}"
    print(label, flush=True)
    Tp = -(-T // G) * G
    g = torch.Generator(device=dev).manual_seed(kb * 100 + vb * 10 + d + T)
    K = (torch.randn(kv, Tp, d, generator=g, device=dev) * torch.exp(torch.randn(kv, 1, d, generator=g, device=dev))
         + 3 * torch.randn(kv, 1, d, generator=g, device=dev))
    V = torch.randn(kv, Tp, d, generator=g, device=dev)
    kc_cfg = P.ChannelQuantConfig(d, kb, G)
    vc_cfg = P.QuantConfig("turboQuant", d, vb, 77)
    kcodes = torch.zeros(kv * Tp * kc_cfg.codeStride, dtype=torch.uint8, device=dev)
    kranges = torch.zeros(kv * (Tp // G) * 2 * d, dtype=torch.float16, device=dev)
    vcodes = torch.zeros(kv * Tp * vc_cfg.codeStride, dtype=torch.uint8, device=dev)
    vscales = torch.zeros(kv * Tp, device=dev)
    for h in range(kv):
        q.enqueuePerChannelEncode(K[h].contiguous(), kcodes, kranges, T, kc_cfg, codesOffset=h * Tp * kc_cfg.codeStride,
                                  rangesOffset=h * (Tp // G) * kc_cfg.rangeStride)
    q.enqueueEncode(V.reshape(-1, d).contiguous(), vcodes, vscales, kv * Tp, vc_cfg)
    Q = torch.randn(kv, nq, d, generator=g, device=dev)
    out = torch.empty(kv, nq, d, device=dev)
    lse = torch.empty(kv, nq, device=dev)
    q.enqueueAttentionDecode(Q, kcodes, kranges, vcodes, vscales, out, T, kc_cfg, vc_cfg, qPerKv=nq, kvHeads=kv,
                             headStride=Tp, lse=lse)
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    kcn = kcodes.cpu().numpy().tobytes()
    krn = kranges.cpu().numpy().view(np.uint16).reshape(kv, Tp // G, 2, d)
    vcn = vcodes.cpu().numpy().tobytes()
    vsn = vscales.cpu().numpy().reshape(kv, Tp)
    Qn = Q.cpu().numpy().astype(np.float64)
    for h in range(kv):
        ck = O.unpack_codes(kcn[h * Tp * kc_cfg.codeStride:(h * Tp + T) * kc_cfg.codeStride], T, d, kb)
        rk = krn[h, :-(-T // G)].view(np.float16)
        cv = O.unpack_codes(vcn[h * Tp * vc_cfg.codeStride:(h * Tp + T) * vc_cfg.codeStride], T, d, vb)
        ro, rl = O.attention_decode_channel_keys(Qn[h], ck, rk, kb, G, cv, vsn[h, :T], "turboQuant", vb,
                                                 1 / math.sqrt(d), 77)
        _check(out[h], lse[h], ro, rl, OUT_REL_L2, LSE_TOL, f"{label} head {h}")


KEY_BIAS_CASES = [
    # (key method, value method, kb, vb, d, nq, kv, T, first position)
    ("turboQuant", "turboQuant", 4, 4, 128, 4, 2, 2000, 0),
    ("polarQuant", "turboQuant", 4, 4, 128, 2, 3, 1500, 17),
    ("turboQuant", "polarQuant", 3, 4, 64, 1, 2, 777, 5),
    ("turboQuant", "turboQuant", 2, 2, 64, 8, 1, 70000, 100),
    ("polarQuant", "polarQuant", 5, 3, 128, 5, 1, 300, 0),
]


@pytest.mark.parametrize("km,vm,kb,vb,d,nq,kv,T,first", KEY_BIAS_CASES)
def test_attention_key_bias(q, km, vm, kb, vb, d, nq, kv, T, first):
    """Keys with a RoPE'd projection bias (Qwen-style, mechanism_eval.py:88-97), encoded with the bias removed
    (pitch_enqueue_encode_key_bias) into a token-major cache; the attention with the same KeyBias scores
    q . (decode(k) + R_t b). Checked against the oracle over the library's codes with R_t b added
    (mechanism_eval.py:113-116), and against float64 attention over the library's own key-bias decode."""
    import torch
    import pitch_amd as P
    from test_gpu_cache_ops import _rope
    dev = q.device
    print(f"attention key bias {km}/{vm} kb={kb} vb={vb} d={d} nq={nq} kv={kv} T={T}", flush=True)
    g = torch.Generator(device=dev).manual_seed(T + d + kb)
    n = T * kv
    bias = (torch.randn(kv, d, generator=g, device=dev) * 6).contiguous()
    cos, sin = _rope(first + T + 3, d, dev)
    t = first + torch.arange(n, device=dev) // kv
    bb = bias[torch.arange(n, device=dev) % kv]
    o = bb * cos[t] + torch.cat([-bb[:, d // 2:], bb[:, :d // 2]], 1) * sin[t]
    K = (torch.randn(n, d, generator=g, device=dev) + o).contiguous()
    V = torch.randn(n, d, generator=g, device=dev)
    kcfg, vcfg = P.QuantConfig(km, d, kb, 0x51), P.QuantConfig(vm, d, vb, 0x52)
    kbias = P.KeyBias(bias, cos, sin, firstPosition=first, heads=kv)
    kc = torch.empty(n * kcfg.codeStride, dtype=torch.uint8, device=dev)
    vc = torch.empty(n * vcfg.codeStride, dtype=torch.uint8, device=dev)
    ks, vs = torch.empty(n, device=dev), torch.empty(n, device=dev)
    q.enqueueEncode(K, kc, ks, n, kcfg, keyBias=kbias)
    q.enqueueEncode(V, vc, vs, n, vcfg)
    Q = torch.randn(kv, nq, d, generator=g, device=dev)
    out = torch.empty(kv, nq, d, device=dev)
    lse = torch.empty(kv, nq, device=dev)
    q.enqueueAttentionDecode(Q, kc, ks, vc, vs, out, T, kcfg, vcfg, qPerKv=nq, kvHeads=kv, tokenStride=kv,
                             headStride=1, lse=lse, keyBias=kbias)
    Kd = torch.empty(n, d, device=dev)
    q.enqueueDecode(kc, ks, Kd, n, kcfg, keyBias=kbias)
    torch.cuda.synchronize()
    Ob = O.key_bias_offsets(bias.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), first, n, kv)
    codes_k = O.unpack_codes(kc.cpu().numpy().tobytes(), n, d, kb)
    codes_v = O.unpack_codes(vc.cpu().numpy().tobytes(), n, d, vb)
    Kr = (O.DECODERS[km](codes_k, ks.cpu().numpy().astype(np.float64), kb, kcfg.seed) + Ob).reshape(T, kv, d)
    Vr = O.DECODERS[vm](codes_v, vs.cpu().numpy().astype(np.float64), vb, vcfg.seed).reshape(T, kv, d)
    Kl = Kd.cpu().numpy().reshape(T, kv, d)
    out, lse, Qn = out.cpu().numpy(), lse.cpu().numpy(), Q.cpu().numpy().astype(np.float64)
    for h in range(kv):
        ro, rl = O.attend(Qn[h], Kr[:, h], Vr[:, h], 1 / math.sqrt(d))
        _check(out[h], lse[h], ro, rl, OUT_REL_L2, LSE_TOL, f"key bias head {h}")
        ro2, rl2 = O.attend(Qn[h], Kl[:, h], Vr[:, h], 1 / math.sqrt(d))
        _check(out[h], lse[h], ro2, rl2, OUT_REL_L2, LSE_TOL, f"key bias head {h} vs library decode")
    # without the key bias the scores lack q . R_t b: the outputs differ (the case the feature exists for)
    plain = torch.empty(kv, nq, d, device=dev)
    q.enqueueAttentionDecode(Q, kc, ks, vc, vs, plain, T, kcfg, vcfg, qPerKv=nq, kvHeads=kv, tokenStride=kv,
                             headStride=1)
    torch.cuda.synchronize()
    assert _rel_l2(plain.cpu().numpy()[0, 0], out[0, 0]) > 1e-3
