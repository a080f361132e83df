"""GPU check of pitch_enqueue_attention_decode_noalloc, the attention entry point that allocates nothing.

It runs the same kernels as pitch_enqueue_attention_decode with the library's per-device scratch array as the
workspace. Two calls in a row, the second with a smaller cache (the scratch keeps the first call's contents),
are each compared with the workspace entry point on the same arguments (the same kernels on the same inputs:
bit for bit) and with the float64 oracle (output within 1e-5 relative L2 per query, log-sum-exp within 1e-5),
through the C ABI with ctypes. A call whose workspace would exceed the scratch is refused before any launch.
"""
import ctypes
import math

import numpy as np
import pytest

from oracle import pitch_oracle as O

pytestmark = pytest.mark.gpu

OUT_REL_L2 = 1e-5
LSE_TOL = 1e-5


def _cache(rng, kv, T, d, bits, lo, hi):
    codes = rng.integers(0, 2 ** bits, (kv, T, d))
    packed = np.frombuffer(b"".join(O.pack_codes(codes[h], bits) for h in range(kv)), np.uint8).reshape(kv, T, -1)
    scales = np.exp(rng.uniform(lo, hi, (kv, T))).astype(np.float32)
    return codes, packed, scales


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()), t.numel() * t.element_size(), 0


def _run(q, kcfg, vcfg, Q, kp, ks, vp, vs, nq, kv, T, noalloc):
    """One call through the C ABI; returns (output, lse) as numpy arrays."""
    import torch
    from pitch_amd import _lib
    dev = q.device
    d = kcfg.dim
    tensors = [torch.from_numpy(Q).to(dev), torch.from_numpy(kp.copy()).to(dev), torch.from_numpy(ks).to(dev),
               torch.from_numpy(vp.copy()).to(dev), torch.from_numpy(vs).to(dev)]
    out = torch.full((kv, nq, d), float("nan"), device=dev)
    lse = torch.full((kv, nq), float("nan"), device=dev)
    desc = _lib.PitchAttentionDescC(nq, kv, T, 1, T, 1.0 / math.sqrt(d), 0)
    args = []
    for t in tensors + [out, lse]:
        args += list(_ptr(t))
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    lib = _lib.load()
    if noalloc:
        rc = lib.pitch_enqueue_attention_decode_noalloc(ctypes.byref(kcfg._c()), ctypes.byref(vcfg._c()),
                                                        ctypes.byref(desc), *args, stream)
    else:
        n = ctypes.c_uint64(0)
        assert lib.pitch_attention_workspace_size(ctypes.byref(kcfg._c()), ctypes.byref(vcfg._c()),
                                                  ctypes.byref(desc), ctypes.byref(n)) == 0
        ws = torch.empty(n.value, dtype=torch.uint8, device=dev)
        rc = lib.pitch_enqueue_attention_decode(ctypes.byref(kcfg._c()), ctypes.byref(vcfg._c()), ctypes.byref(desc),
                                                *args, *_ptr(ws)[:2], stream)
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    return out.cpu().numpy(), lse.cpu().numpy()


def _case(q, seed, kmeth, vmeth, kb, vb, d, nq, kv, T):
    import pitch_amd as P
    print(f"noalloc attention K {kmeth} b{kb} V {vmeth} b{vb} d={d} nq={nq} kv={kv} T={T}", flush=True)
    rng = np.random.default_rng(seed)
    kc, kp, ks = _cache(rng, kv, T, d, kb, 1.5, 3.0)
    vc, vp, vs = _cache(rng, kv, T, d, vb, -1.0, 1.0)
    Q = rng.standard_normal((kv, nq, d)).astype(np.float32)
    kcfg, vcfg = P.QuantConfig(kmeth, d, kb, 11), P.QuantConfig(vmeth, d, vb, 22)
    out_n, lse_n = _run(q, kcfg, vcfg, Q, kp, ks, vp, vs, nq, kv, T, noalloc=True)
    out_w, lse_w = _run(q, kcfg, vcfg, Q, kp, ks, vp, vs, nq, kv, T, noalloc=False)
    assert np.array_equal(out_n.view(np.uint32), out_w.view(np.uint32))
    assert np.array_equal(lse_n.view(np.uint32), lse_w.view(np.uint32))
    for h in range(kv):
        ro, rl = O.attention_decode(Q[h].astype(np.float64), kc[h], ks[h], vc[h], vs[h], kmeth, kb, vmeth, vb,
                                    1 / math.sqrt(d), 11, 22)
        for i in range(nq):
            e = np.linalg.norm(out_n[h, i] - ro[i]) / np.linalg.norm(ro[i])
            assert e < OUT_REL_L2, (h, i, e)
        err = np.abs(lse_n[h].astype(np.float64) - rl) / np.maximum(1.0, np.abs(rl))
        assert err.max() < LSE_TOL


def test_noalloc_two_calls_second_smaller(q):
    # first call: two chunked KV heads at d = 128 (fused scores-and-values kernel); second: a smaller d = 64 call
    # with unequal key and value widths (the separate score and value kernels, which keep weights in the scratch)
    _case(q, 1, "turboQuant", "turboQuant", 4, 4, 128, 4, 2, 9000)
    _case(q, 2, "polarQuant", "turboQuant", 5, 2, 64, 2, 1, 700)


def test_noalloc_refuses_workspace_beyond_scratch(q):
    """8 KV heads x 8 query heads x 2^20 tokens needs far more than 32 MiB of workspace: refused before any launch
    (the buffers are sized for the check only; nothing is read)."""
    import torch
    import pitch_amd as P
    from pitch_amd import _lib
    cfg = P.QuantConfig("turboQuant", 64, 2)
    kv, nq, T = 8, 8, 1 << 20
    n = ctypes.c_uint64(0)
    desc = _lib.PitchAttentionDescC(nq, kv, T, 1, T, 0.125, 0)
    lib = _lib.load()
    assert lib.pitch_attention_workspace_size(ctypes.byref(cfg._c()), ctypes.byref(cfg._c()), ctypes.byref(desc),
                                              ctypes.byref(n)) == 0
    assert n.value > _lib.NOALLOC_SCRATCH_BYTES
    dev = q.device
    qt = torch.zeros(kv, nq, 64, device=dev)
    codes = torch.zeros(kv * T * cfg.codeStride, dtype=torch.uint8, device=dev)
    scales = torch.zeros(kv * T, device=dev)
    out = torch.zeros(kv, nq, 64, device=dev)
    args = []
    for t in (qt, codes, scales, codes, scales, out):
        args += list(_ptr(t))
    args += [None, 0, 0]
    rc = lib.pitch_enqueue_attention_decode_noalloc(ctypes.byref(cfg._c()), ctypes.byref(cfg._c()),
                                                    ctypes.byref(desc), *args, None)
    assert rc == _lib.ERR_INVALID_INPUT and "allocation-free" in _lib.last_error()
    torch.cuda.synchronize()
