#!/usr/bin/env python3
"""Benchmark of the MI355X KV-cache codec (headline: BASELINE config 2 full-cache decode).

    python bench.py [--steps K] [--warmup W] [--bits 4] [--sets 8] [--extras] [--full] [--no-cpu]

A step is one full-cache decode of the GPT-2-small-shaped value cache (32768 tokens x 12 heads x d=64,
393,216 vectors, TurboQuant b=4, fp32 token-major) with codes, norms and the output already resident in
HBM. Steps rotate over --sets independent buffer sets (default 8, ~0.9 GB) so the 256 MB Infinity Cache
cannot serve them. Every timed measurement follows at least W warm-up calls and at least 0.25 s of calls. value = algorithmic bytes per step / time per step, with algorithmic bytes
n * (4d + codeStride + 4). One JSON line is printed; --extras adds the other BASELINE configs
(bulk encode, append-encode latency, KIVI, d=128 TurboQuant/PolarQuant), float16/bfloat16 caches and
decode-step attention over compressed caches under "extra", and --full adds config 5 (Llama-3-8B long
context, ~80 GB of buffers) and the d=1024 sweep.

Before timing, encode output is checked against the CPU oracle on a sample (codes may differ only at
near-boundary coordinates); the benchmark refuses to report otherwise.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_GBPS = 8000.0
METRIC = "codec GB/s (fp32 in/out + codes) and % of HBM peak; vectors/s at d=64/128"


def per_vector_bytes(d: int, b: int) -> int:
    return 4 * d + ((d * b + 31) // 32) * 4 + 4


def per_vector_bytes16(d: int, b: int) -> int:
    """Per-vector algorithmic bytes with float16 / bfloat16 vectors: 2d + codeStride + 4."""
    return 2 * d + ((d * b + 31) // 32) * 4 + 4


def kivi_bytes(n: int, d: int, b: int, G: int, heads: int = 1, elem: int = 4) -> int:
    """n tokens per head: n*(elem*d + codeStride) + groups * 4d per head (elem = bytes per key element)."""
    cs = ((d * b + 31) // 32) * 4
    return heads * (n * (elem * d + cs) + ((n + G - 1) // G) * 4 * d)


WARMUP_S = 0.25  # minimum warm-up per timed measurement, as the reference's benchmarks (BenchmarkSuite.swift:150-185)


class Timer:
    """HIP events on the stream the codec launches on (torch's current stream)."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.current_stream()

    def time(self, fn, steps: int, warmup: int) -> float:
        """Average milliseconds per call of fn(i) over `steps` calls, after at least `warmup` calls and at least
        WARMUP_S seconds of calls: the GPU's clocks take milliseconds to ramp up, so a warm-up of a few short
        calls under-reports sustained throughput by up to 20 %."""
        torch = self.torch
        i, t0 = 0, time.perf_counter()
        while i < warmup or time.perf_counter() - t0 < WARMUP_S:
            fn(i)
            i += 1
            if i % 64 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        warmup = i
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for i in range(steps):
            fn(warmup + i)
        end.record(self.stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps


def profiled_traffic(bits: int):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 PMC summary, if present."""
    f = ROOT / "profiles" / "vec_decode_d64_b4_config2_hbm_traffic.md"
    if bits != 4 or not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":")[1])
    return None


def student_t(torch, shape, nu, gen, device):
    """Student-t(nu) = N(0,1) / sqrt(chi2(nu) / nu), generated on the device.

    The Gamma sampler takes no generator and draws from torch's default CUDA generator, so that one is
    seeded from gen first: the same seed gives the same values in every run."""
    z = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    seed = int(torch.randint(0, 2**62, (1,), generator=gen, device=device).item())
    torch.cuda.manual_seed(seed)
    g = torch.distributions.Gamma(torch.tensor(nu / 2.0, device=device), torch.tensor(0.5, device=device))
    chi2 = g.sample(shape)
    return z / torch.sqrt(chi2 / nu)


def gpt2_values(torch, gen, device, tokens=32768, heads=12, d=64):
    """Config 2: Student-t (nu=5) values scaled per head by log-uniform factors in [0.5, 4]."""
    x = student_t(torch, (tokens, heads, d), 5.0, gen, device)
    f = torch.exp(torch.empty(heads, device=device).uniform_(math.log(0.5), math.log(4.0), generator=gen))
    return (x * f.view(1, heads, 1)).contiguous()


def biased_keys(torch, gen, device, heads, tokens, d, scale_sigma=1.0, outliers=4, outlier_x=20.0, bias_sd=3.0):
    """Configs 3-5 keys: N(0,1) * per-channel log-normal scales, outlier channels, per-head bias."""
    x = torch.randn((heads, tokens, d), generator=gen, device=device)
    s = torch.exp(torch.randn((heads, 1, d), generator=gen, device=device) * scale_sigma)
    for h in range(heads):
        idx = torch.randperm(d, generator=torch.Generator().manual_seed(1000 + h))[:outliers].to(device)
        s[h, 0, idx] *= outlier_x
    bias = torch.randn((heads, 1, d), generator=gen, device=device) * bias_sd
    return (x * s + bias).contiguous()


def parity_gate(torch, q, P, O, x_host, method, d, b, label):
    """Encode a sample on the GPU and compare with the oracle (pytorch_mps_benchmark.py:82-104 pattern)."""
    import numpy as np
    X = x_host.reshape(-1, d)
    cfg = P.QuantConfig(method, d, b)
    ours = q.encode(X.reshape(-1), config=cfg)
    codes, scales = O.ENCODERS[method](X.astype(np.float64), b)
    a = O.unpack_codes(ours.codes, X.shape[0], d, b)
    diff = a != codes
    if diff.any():
        band = (O.turbo_near_boundary(O.turbo_rotated(X.astype(np.float64)), b) if method == "turboQuant"
                else O.polar_near_boundary(X.astype(np.float64), b))
        if (diff & ~band).any():
            raise SystemExit(f"parity gate failed for {label}: {int((diff & ~band).sum())} codes differ")
    return int(diff.sum())


def cpu_baseline(O, x_host, d, b, seconds=12.0):
    """Oracle (numpy, float64 spec semantics, 1 thread) full decode over a bounded sample."""
    import numpy as np
    X = x_host.reshape(-1, d).astype(np.float64)
    n = X.shape[0]
    codes, norms = O.turbo_encode(X, b)
    norms32 = np.asarray(norms, np.float32).astype(np.float64)
    O.turbo_decode(codes[:1024], norms32[:1024], b)  # warm-up
    runs, t0 = 0, time.perf_counter()
    times = []
    while time.perf_counter() - t0 < seconds or runs < 3:
        t1 = time.perf_counter()
        O.turbo_decode(codes, norms32, b)
        times.append(time.perf_counter() - t1)
        runs += 1
    t = sorted(times)[len(times) // 2]
    return {"value": round(n * per_vector_bytes(d, b) / t / 1e9, 4), "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"oracle/pitch_oracle.py turbo_decode of {n} vectors d={d} b={b} (float64, numpy, "
                      f"1 thread), median of {runs} runs: {t * 1e3:.1f} ms; vectors/s {n / t:.3e}",
            "host_cpus": {"affinity": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count()}}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--sets", type=int, default=8)
    ap.add_argument("--extras", action="store_true")
    ap.add_argument("--full", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calib", action="store_true", help="also run a plain 1 GiB device copy (PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the codec needs no collective and this build measures one "
              f"GPU's share (got --gpus {args.gpus})", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    import pitch_amd as P
    from oracle import pitch_oracle as O

    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q = P.PITCH(device=dev)
    timer = Timer(torch)
    gen = torch.Generator(device=dev).manual_seed(2)

    # ---------------- headline: config 2 full-cache decode
    d, b, n = 64, args.bits, 32768 * 12
    cfg = P.QuantConfig("turboQuant", d, b)
    print(f"# generating config 2 ({args.sets} buffer sets)", file=sys.stderr, flush=True)
    x = gpt2_values(torch, gen, dev)
    gate_diffs = parity_gate(torch, q, P, O, x.reshape(-1, d)[:8192].cpu().numpy(), "turboQuant", d, b, "config2")
    sets = []
    for s in range(args.sets):
        xs = x if s == 0 else gpt2_values(torch, gen, dev)
        codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
        norms = torch.empty(n, dtype=torch.float32, device=dev)
        q.enqueueEncode(xs, codes, norms, n, cfg)
        out = torch.empty((n, d), dtype=torch.float32, device=dev)
        sets.append((codes, norms, out))
        if s:
            del xs
    torch.cuda.synchronize()
    x_host = x.reshape(-1, d).cpu().numpy()

    def dec_step(i):
        c, s_, o = sets[i % len(sets)]
        q.enqueueDecode(c, s_, o, n, cfg)

    print("# timing config 2 decode", file=sys.stderr, flush=True)
    ms = timer.time(dec_step, args.steps, args.warmup)
    nbytes = n * per_vector_bytes(d, b)
    gbps = nbytes / (ms * 1e-3) / 1e9
    traffic = profiled_traffic(b)
    # decode of set 0 vs the oracle on a sample (the timed output is the product)
    c0, s0, o0 = sets[0]
    samp = np.random.default_rng(0).choice(n, 4096, replace=False)
    codes_np = O.unpack_codes(c0.cpu().numpy().tobytes(), n, d, b)[samp]
    ref = O.turbo_decode(codes_np, s0.cpu().numpy()[samp].astype(np.float64), b)
    got = o0.cpu().numpy()[samp].astype(np.float64)
    rel = float(np.max(np.sqrt(((got - ref) ** 2).sum(1) / (ref ** 2).sum(1))))
    if rel > 1e-5:
        print(f"decode parity failed: max rel L2 {rel}", file=sys.stderr)
        return 1

    result = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: Student-t(nu=5) values x per-head log-uniform[0.5,4] factors, generated on device",
        "config": {"workload": "config2 full-cache decode: TurboQuant b=%d, 32768 tokens x 12 heads x d=64 "
                               "(393,216 vectors), fp32 token-major, %d rotated buffer sets" % (b, args.sets),
                   "method": "turboQuant", "dim": d, "bits": b, "vectors": n, "bytes_per_step": nbytes},
        "vectors_per_s": round(n / (ms * 1e-3), 1),
        "pct_of_hbm_peak": round(100 * gbps / PEAK_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_GBPS, 4), "traffic": traffic,
                     "kernel": f"pitch::vec_decode<64, {b}, false, 0, false>",
                     "kernel_us_per_launch": round(ms * 1e3, 3),
                     "algorithmic_bytes_per_launch": nbytes,
                     "traffic_source": ("profiles/vec_decode_d64_b4_config2_hbm_traffic.md (rocprofv3 FETCH_SIZE x2 "
                                        "+ WRITE_SIZE x1, scaled by a 1 GiB copy)") if traffic else None},
        "parity": {"encode_code_diffs_near_boundary": gate_diffs, "decode_max_rel_l2": rel},
    }

    extra = {}
    if args.extras or args.full:
        extra.update(run_extras(torch, q, P, O, timer, gen, dev, args, x, sets))
    if args.full:
        extra.update(run_full(torch, q, P, timer, gen, dev, args))
    if extra:
        result["extra"] = extra
    if args.copy_calib:
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        bb = torch.empty_like(a)
        for _ in range(3):
            bb.copy_(a)
        torch.cuda.synchronize()
        result["copy_calibration"] = {"bytes_read": a.numel() * 4, "bytes_written": a.numel() * 4, "calls": 3}
    if not args.no_cpu:
        print("# CPU baseline (oracle)", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(O, x_host, d, b)
    print(json.dumps(result), flush=True)
    return 0


def run_extras(torch, q, P, O, timer, gen, dev, args, x, sets) -> dict:
    import numpy as np
    out = {}
    steps, warm = max(20, args.steps // 4), 5
    d, n = 64, 32768 * 12
    # config 2 decode at b = 2, 3 and bulk encode at b = 2, 3, 4
    for b in (2, 3, 4):
        cfg = P.QuantConfig("turboQuant", d, b)
        bufs = []
        for s in range(args.sets):
            xs = x if s == 0 else gpt2_values(torch, gen, dev)
            c = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
            nm = torch.empty(n, dtype=torch.float32, device=dev)
            q.enqueueEncode(xs, c, nm, n, cfg)
            bufs.append((xs, c, nm, torch.empty((n, d), dtype=torch.float32, device=dev)))
        ms_enc = timer.time(lambda i: q.enqueueEncode(bufs[i % len(bufs)][0], bufs[i % len(bufs)][1],
                                                      bufs[i % len(bufs)][2], n, cfg), steps, warm)
        ms_dec = timer.time(lambda i: q.enqueueDecode(bufs[i % len(bufs)][1], bufs[i % len(bufs)][2],
                                                      bufs[i % len(bufs)][3], n, cfg), steps, warm)
        nb = n * per_vector_bytes(d, b)
        out[f"cfg2_tq_d64_b{b}"] = {"encode_gbps": round(nb / ms_enc / 1e6, 1), "decode_gbps": round(nb / ms_dec / 1e6, 1),
                                    "encode_ms": round(ms_enc, 5), "decode_ms": round(ms_dec, 5),
                                    "encode_pct_peak": round(nb / ms_enc / 1e6 / PEAK_GBPS * 100, 1),
                                    "decode_pct_peak": round(nb / ms_dec / 1e6 / PEAK_GBPS * 100, 1)}
        del bufs
    # append-encode latency: 12 vectors per step at codesOffset = t*12*cs
    cfg = P.QuantConfig("turboQuant", d, 3)
    xs = x.reshape(-1, 12, d)
    codes = torch.empty(32768 * 12 * cfg.codeStride, dtype=torch.uint8, device=dev)
    norms = torch.empty(32768 * 12, dtype=torch.float32, device=dev)

    def app(i):
        t = i % 32768
        q.enqueueEncode(x, codes, norms, 12, cfg, inputOffset=t * 12 * d * 4, codesOffset=t * 12 * cfg.codeStride,
                        scalesOffset=t * 12 * 4)

    ms_app = timer.time(app, 500, 50)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(500):
        app(i)
        torch.cuda.current_stream().synchronize()
    wall = (time.perf_counter() - t0) / 500 * 1e6
    out["cfg2_append_encode_12vec"] = {"gpu_us_per_call_backtoback": round(ms_app * 1e3, 2),
                                       "wall_us_per_call_synchronous": round(wall, 2)}
    # config 3: KIVI keys, Llama-3.2-1B shape (8 heads x 32768 tokens x 64), G=64, b=4
    keys = biased_keys(torch, gen, dev, 8, 32768, 64)
    ccfg = P.ChannelQuantConfig(64, 4, 64)
    nt = 32768
    kbufs = []
    for s in range(args.sets):
        kk = keys if s == 0 else biased_keys(torch, gen, dev, 8, 32768, 64)
        c = torch.empty(8 * nt * ccfg.codeStride, dtype=torch.uint8, device=dev)
        r = torch.empty(8 * ccfg.groupCount(nt) * 2 * 64, dtype=torch.float16, device=dev)
        kbufs.append((kk, c, r, torch.empty_like(kk)))
    # one call over all heads: groups never cross a head (32768 % 64 == 0)
    ms_ke = timer.time(lambda i: q.enqueuePerChannelEncode(kbufs[i % len(kbufs)][0], kbufs[i % len(kbufs)][1],
                                                           kbufs[i % len(kbufs)][2], 8 * nt, ccfg), steps, warm)
    ms_kd = timer.time(lambda i: q.enqueuePerChannelDecode(kbufs[i % len(kbufs)][1], kbufs[i % len(kbufs)][2],
                                                           kbufs[i % len(kbufs)][3], 8 * nt, ccfg), steps, warm)
    kb = kivi_bytes(nt, 64, 4, 64, heads=8)
    # parity gate for KIVI: bit-exact on head 0
    k0 = keys[0].cpu().numpy()
    codes_ref, ranges_ref = O.channel_encode(k0, 4, 64)
    c0 = kbufs[0][1][: nt * ccfg.codeStride].cpu().numpy().tobytes()
    r0 = kbufs[0][2][: ccfg.groupCount(nt) * 128].cpu().numpy()
    kivi_exact = (c0 == O.pack_codes(codes_ref, 4)) and np.array_equal(r0.view(np.uint16),
                                                                      ranges_ref.reshape(-1).view(np.uint16))
    out["cfg3_kivi_d64_b4_G64"] = {"encode_gbps": round(kb / ms_ke / 1e6, 1), "decode_gbps": round(kb / ms_kd / 1e6, 1),
                                   "encode_ms": round(ms_ke, 5), "decode_ms": round(ms_kd, 5),
                                   "encode_pct_peak": round(kb / ms_ke / 1e6 / PEAK_GBPS * 100, 1),
                                   "decode_pct_peak": round(kb / ms_kd / 1e6 / PEAK_GBPS * 100, 1),
                                   "bit_exact_head0": bool(kivi_exact)}
    del kbufs, keys
    # config 4: Qwen2.5-1.5B shape d=128, 28 L x 2 h x 16384 tokens, TurboQuant and PolarQuant b=4
    n4 = 28 * 2 * 16384
    keys4 = biased_keys(torch, gen, dev, 56, 16384, 128, scale_sigma=0.0, outliers=2, outlier_x=30.0,
                        bias_sd=5.0).reshape(n4, 128)
    for method in ("turboQuant", "polarQuant"):
        cfg4 = P.QuantConfig(method, 128, 4)
        c = torch.empty(n4 * cfg4.codeStride, dtype=torch.uint8, device=dev)
        s_ = torch.empty(n4, dtype=torch.float32, device=dev)
        o = torch.empty_like(keys4)
        ms_e = timer.time(lambda i: q.enqueueEncode(keys4, c, s_, n4, cfg4), steps, warm)
        ms_d = timer.time(lambda i: q.enqueueDecode(c, s_, o, n4, cfg4), steps, warm)
        nb = n4 * per_vector_bytes(128, 4)
        diffs = parity_gate(torch, q, P, O, keys4[:4096].cpu().numpy(), method, 128, 4, f"config4 {method}")
        out[f"cfg4_{method}_d128_b4"] = {"encode_gbps": round(nb / ms_e / 1e6, 1), "decode_gbps": round(nb / ms_d / 1e6, 1),
                                         "encode_ms": round(ms_e, 5), "decode_ms": round(ms_d, 5),
                                         "encode_pct_peak": round(nb / ms_e / 1e6 / PEAK_GBPS * 100, 1),
                                         "decode_pct_peak": round(nb / ms_d / 1e6 / PEAK_GBPS * 100, 1),
                                         "vectors_per_s_decode": round(n4 / ms_d * 1e3, 1),
                                         "parity_code_diffs_near_boundary": diffs}
        del c, s_, o
    out.update(run_io16(torch, q, P, timer, gen, dev, args, x, keys4))
    out.update(run_attention(torch, q, P, O, timer, gen, dev, args))
    out.update(run_key_bias(torch, q, P, timer, gen, dev, args))
    return out


def run_key_bias(torch, q, P, timer, gen, dev, args) -> dict:
    """Config 4 (Qwen2.5-1.5B: 28 layers x 2 KV heads x 16384 tokens x d=128, TurboQuant b=4), one call per layer
    as a model makes them, with and without the RoPE'd key-bias removal (Qwen's key projection has a bias).
    Algorithmic bytes count the vectors, codes and scales (the bias and RoPE tables are extra reads)."""
    out = {}
    L, H, T, d = 28, 2, 16384, 128
    n = H * T
    cfg = P.QuantConfig("turboQuant", d, 4)
    inv = 1.0 / 1e6 ** (torch.arange(0, d, 2, dtype=torch.float64, device=dev) / d)
    ang = torch.arange(T, dtype=torch.float64, device=dev)[:, None] * inv[None, :]
    cos = torch.cat([torch.cos(ang)] * 2, 1).float().contiguous()
    sin = torch.cat([torch.sin(ang)] * 2, 1).float().contiguous()
    layers = []
    for _ in range(L):
        x = torch.randn(n, d, generator=gen, device=dev)
        c = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
        s_ = torch.empty(n, device=dev)
        kb = P.KeyBias(torch.randn(H, d, generator=gen, device=dev) * 8, cos, sin, 0, H)
        layers.append((x, c, s_, torch.empty_like(x), kb))
    nb = n * per_vector_bytes(d, 4)
    steps = L * max(4, args.steps // 40)
    for name, use in (("plain", False), ("key_bias", True)):
        ms_e = timer.time(lambda i: q.enqueueEncode(layers[i % L][0], layers[i % L][1], layers[i % L][2], n, cfg,
                                                    keyBias=layers[i % L][4] if use else None), steps, L)
        ms_d = timer.time(lambda i: q.enqueueDecode(layers[i % L][1], layers[i % L][2], layers[i % L][3], n, cfg,
                                                    keyBias=layers[i % L][4] if use else None), steps, L)
        out[f"cfg4_qwen_layer_tq_d128_b4_{name}"] = {"vectors_per_call": n, "encode_us": round(ms_e * 1e3, 2),
                                                     "decode_us": round(ms_d * 1e3, 2),
                                                     "encode_gbps": round(nb / ms_e / 1e6, 1),
                                                     "decode_gbps": round(nb / ms_d / 1e6, 1)}
    del layers
    torch.cuda.empty_cache()
    return out


def run_attention(torch, q, P, O, timer, gen, dev, args) -> dict:
    """Decode-step attention directly over TurboQuant b=4 K and V caches (pitch_enqueue_attention_decode),
    against decoding both caches to fp32 and attending with torch (the reference's flow: decode, then attend).
    Algorithmic bytes per call are the compressed caches' codes and scales: kv_heads * T * 2 * (cs + 4)."""
    import numpy as np
    out = {}
    steps, warm = max(20, args.steps // 4), 5
    for label, kv, nq, d, T in (("cfg2_gpt2_attention_T32768", 12, 1, 64, 32768),
                                ("cfg5_llama3_8b_layer_attention_T32768", 8, 4, 128, 32768),
                                ("cfg5_llama3_8b_layer_attention_T131072", 8, 4, 128, 131072)):
        cfg = P.QuantConfig("turboQuant", d, 4)
        n = kv * T
        K = torch.randn(kv, T, d, generator=gen, device=dev)
        V = torch.randn(kv, T, d, generator=gen, device=dev)
        kc = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
        vc = torch.empty_like(kc)
        ks = torch.empty(n, device=dev)
        vs = torch.empty_like(ks)
        q.enqueueEncode(K, kc, ks, n, cfg)
        q.enqueueEncode(V, vc, vs, n, cfg)
        del K, V
        Q = torch.randn(kv, nq, d, generator=gen, device=dev)
        o = torch.empty(kv, nq, d, device=dev)
        lse = torch.empty(kv, nq, device=dev)
        ws = torch.empty(P.attention_workspace_bytes(cfg, cfg, T, nq, kv), dtype=torch.uint8, device=dev)
        ms = timer.time(lambda i: q.enqueueAttentionDecode(Q, kc, ks, vc, vs, o, T, cfg, qPerKv=nq, kvHeads=kv,
                                                           lse=lse, workspace=ws), steps, warm)
        Kd = torch.empty(n, d, device=dev)
        Vd = torch.empty(n, d, device=dev)

        def decode_then_attend(i):
            q.enqueueDecode(kc, ks, Kd, n, cfg)
            q.enqueueDecode(vc, vs, Vd, n, cfg)
            S = torch.bmm(Q, Kd.view(kv, T, d).transpose(1, 2).contiguous()) / math.sqrt(d)
            return torch.bmm(torch.softmax(S, -1), Vd.view(kv, T, d))

        ms_b = timer.time(decode_then_attend, max(5, steps // 4), 2)
        # parity: head 0 against the float64 oracle over the same codes
        torch.cuda.synchronize()
        cs = cfg.codeStride
        ck = O.unpack_codes(kc[:T * cs].cpu().numpy().tobytes(), T, d, 4)
        cv = O.unpack_codes(vc[:T * cs].cpu().numpy().tobytes(), T, d, 4)
        ro, rl = O.attention_decode(Q[0].cpu().numpy().astype(np.float64), ck, ks[:T].cpu().numpy(), cv,
                                    vs[:T].cpu().numpy(), "turboQuant", 4, "turboQuant", 4, 1 / math.sqrt(d))
        got = o[0].cpu().numpy().astype(np.float64)
        rel = float(max(np.linalg.norm(got[i] - ro[i]) / np.linalg.norm(ro[i]) for i in range(nq)))
        if rel > 1e-5:
            raise SystemExit(f"attention parity failed for {label}: rel L2 {rel}")
        nb = n * 2 * (cs + 4)
        out[label] = {"kv_heads": kv, "q_per_kv": nq, "dim": d, "tokens": T, "ms": round(ms, 5),
                      "cache_tokens_per_s": round(n / ms * 1e3, 1), "codes_gbps": round(nb / ms / 1e6, 1),
                      "codes_pct_peak": round(nb / ms / 1e6 / PEAK_GBPS * 100, 1),
                      "decode_then_attend_ms": round(ms_b, 4), "speedup_vs_decode_then_attend": round(ms_b / ms, 2),
                      "parity_max_rel_l2_head0": rel}
        del kc, vc, ks, vs, Kd, Vd, ws
        torch.cuda.empty_cache()
    # per-channel keys (KIVI b=4, G=64) with TurboQuant b=4 values: the reference's recommended configuration
    kv, nq, d, T, G = 8, 4, 128, 32768, 64
    kcfg, vcfg = P.ChannelQuantConfig(d, 4, G), P.QuantConfig("turboQuant", d, 4)
    K = biased_keys(torch, gen, dev, kv, T, d)
    V = torch.randn(kv * T, d, generator=gen, device=dev)
    kc = torch.empty(kv * T * kcfg.codeStride, dtype=torch.uint8, device=dev)
    kr = torch.empty(kv * (T // G) * 2 * d, dtype=torch.float16, device=dev)
    vc = torch.empty(kv * T * vcfg.codeStride, dtype=torch.uint8, device=dev)
    vs = torch.empty(kv * T, device=dev)
    for h in range(kv):
        q.enqueuePerChannelEncode(K[h], kc, kr, T, kcfg, codesOffset=h * T * kcfg.codeStride,
                                  rangesOffset=h * (T // G) * kcfg.rangeStride)
    q.enqueueEncode(V, vc, vs, kv * T, vcfg)
    Q = torch.randn(kv, nq, d, generator=gen, device=dev)
    o = torch.empty(kv, nq, d, device=dev)
    ws = torch.empty(P.attention_workspace_bytes(vcfg, vcfg, T, nq, kv), dtype=torch.uint8, device=dev)
    ms = timer.time(lambda i: q.enqueueAttentionDecode(Q, kc, kr, vc, vs, o, T, kcfg, vcfg, qPerKv=nq, kvHeads=kv,
                                                       headStride=T, workspace=ws), steps, warm)
    Kd = torch.empty(kv * T, d, device=dev)
    Vd = torch.empty(kv * T, d, device=dev)

    def decode_then_attend_kivi(i):
        for h in range(kv):
            q.enqueuePerChannelDecode(kc, kr, Kd, T, kcfg, codesOffset=h * T * kcfg.codeStride,
                                      rangesOffset=h * (T // G) * kcfg.rangeStride, outputOffset=h * T * d * 4)
        q.enqueueDecode(vc, vs, Vd, kv * T, vcfg)
        S = torch.bmm(Q, Kd.view(kv, T, d).transpose(1, 2).contiguous()) / math.sqrt(d)
        return torch.bmm(torch.softmax(S, -1), Vd.view(kv, T, d))

    ms_b = timer.time(decode_then_attend_kivi, max(5, steps // 4), 2)
    torch.cuda.synchronize()
    ck = O.unpack_codes(kc[:T * kcfg.codeStride].cpu().numpy().tobytes(), T, d, 4)
    rk = kr[:(T // G) * 2 * d].cpu().numpy().reshape(T // G, 2, d)
    cv = O.unpack_codes(vc[:T * vcfg.codeStride].cpu().numpy().tobytes(), T, d, 4)
    ro, _ = O.attention_decode_channel_keys(Q[0].cpu().numpy().astype(np.float64), ck, rk, 4, G, cv,
                                            vs[:T].cpu().numpy(), "turboQuant", 4, 1 / math.sqrt(d))
    got = o[0].cpu().numpy().astype(np.float64)
    rel = float(max(np.linalg.norm(got[i] - ro[i]) / np.linalg.norm(ro[i]) for i in range(nq)))
    if rel > 1e-5:
        raise SystemExit(f"attention parity failed for per-channel keys: rel L2 {rel}")
    nb = kv * T * (kcfg.codeStride + vcfg.codeStride + 4) + kv * (T // G) * 4 * d
    out["cfg5_llama3_8b_layer_attention_kivi_keys_T32768"] = {
        "kv_heads": kv, "q_per_kv": nq, "dim": d, "tokens": T, "key_group": G, "ms": round(ms, 5),
        "cache_tokens_per_s": round(kv * T / ms * 1e3, 1), "codes_gbps": round(nb / ms / 1e6, 1),
        "decode_then_attend_ms": round(ms_b, 4), "speedup_vs_decode_then_attend": round(ms_b / ms, 2),
        "parity_max_rel_l2_head0": rel}
    del K, V, kc, kr, vc, vs, Kd, Vd, ws
    torch.cuda.empty_cache()
    return out


def run_io16(torch, q, P, timer, gen, dev, args, x, keys4) -> dict:
    """float16 / bfloat16 cache I/O: config 2 (TurboQuant d=64 b=4), config 4 (TurboQuant d=128 b=4) and
    config 3 KIVI, encode and decode, with algorithmic bytes counted at 2 bytes per element."""
    out = {}
    steps, warm = max(20, args.steps // 4), 5
    for io in ("float16", "bfloat16"):
        dt = getattr(torch, io)
        for label, src, d in (("cfg2_tq_d64_b4", x.reshape(-1, 64), 64), ("cfg4_tq_d128_b4", keys4, 128)):
            n = src.shape[0]
            cfg = P.QuantConfig("turboQuant", d, 4)
            # enough buffer sets that the inputs of consecutive calls never fit the 256 MB Infinity Cache
            nsets = args.sets if d == 64 else 2
            bufs = []
            for s in range(nsets):
                xs = torch.roll(src, s * 997, 0).to(dt).contiguous()
                c = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
                nm = torch.empty(n, dtype=torch.float32, device=dev)
                q.enqueueEncode(xs, c, nm, n, cfg)
                bufs.append((xs, c, nm, torch.empty((n, d), dtype=dt, device=dev)))
            ms_e = timer.time(lambda i: q.enqueueEncode(bufs[i % nsets][0], bufs[i % nsets][1], bufs[i % nsets][2],
                                                        n, cfg), steps, warm)
            ms_d = timer.time(lambda i: q.enqueueDecode(bufs[i % nsets][1], bufs[i % nsets][2], bufs[i % nsets][3],
                                                        n, cfg), steps, warm)
            nb = n * per_vector_bytes16(d, 4)
            out[f"{label}_{io}"] = {"encode_gbps": round(nb / ms_e / 1e6, 1), "decode_gbps": round(nb / ms_d / 1e6, 1),
                                    "encode_ms": round(ms_e, 5), "decode_ms": round(ms_d, 5),
                                    "encode_pct_peak": round(nb / ms_e / 1e6 / PEAK_GBPS * 100, 1),
                                    "decode_pct_peak": round(nb / ms_d / 1e6 / PEAK_GBPS * 100, 1),
                                    "vectors_per_s_decode": round(n / ms_d * 1e3, 1)}
            del bufs
        ccfg = P.ChannelQuantConfig(64, 4, 64)
        nt = 8 * 32768
        kb_list = []
        for s in range(args.sets):
            kk = biased_keys(torch, gen, dev, 8, 32768, 64).reshape(nt, 64).to(dt).contiguous()
            c = torch.empty(nt * ccfg.codeStride, dtype=torch.uint8, device=dev)
            r = torch.empty(ccfg.groupCount(nt) * 2 * 64, dtype=torch.float16, device=dev)
            kb_list.append((kk, c, r, torch.empty_like(kk)))
        ms_e = timer.time(lambda i: q.enqueuePerChannelEncode(kb_list[i % len(kb_list)][0], kb_list[i % len(kb_list)][1],
                                                              kb_list[i % len(kb_list)][2], nt, ccfg), steps, warm)
        ms_d = timer.time(lambda i: q.enqueuePerChannelDecode(kb_list[i % len(kb_list)][1], kb_list[i % len(kb_list)][2],
                                                              kb_list[i % len(kb_list)][3], nt, ccfg), steps, warm)
        kb = kivi_bytes(nt, 64, 4, 64, elem=2)
        out[f"cfg3_kivi_d64_b4_G64_{io}"] = {"encode_gbps": round(kb / ms_e / 1e6, 1),
                                              "decode_gbps": round(kb / ms_d / 1e6, 1),
                                              "encode_ms": round(ms_e, 5), "decode_ms": round(ms_d, 5),
                                              "encode_pct_peak": round(kb / ms_e / 1e6 / PEAK_GBPS * 100, 1),
                                              "decode_pct_peak": round(kb / ms_d / 1e6 / PEAK_GBPS * 100, 1)}
        del kb_list
    return out


def run_full(torch, q, P, timer, gen, dev, args) -> dict:
    """Config 5 (per-layer slices of a 32 L x 8 h x 131072 x 128 cache) and the d=1024 sweep."""
    out = {}
    L, H, T, d = 32, 8, 131072, 128
    n_layer = H * T
    # values: TurboQuant b=3, full-cache decode (all layers in one call)
    cfg = P.QuantConfig("turboQuant", d, 3)
    n = L * n_layer
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    norms = torch.empty(n, dtype=torch.float32, device=dev)
    for layer in range(L):
        v = student_t(torch, (n_layer, d), 5.0, gen, dev)
        q.enqueueEncode(v, codes, norms, n_layer, cfg, codesOffset=layer * n_layer * cfg.codeStride,
                        scalesOffset=layer * n_layer * 4)
        del v
    outv = torch.empty((n, d), dtype=torch.float32, device=dev)
    ms = timer.time(lambda i: q.enqueueDecode(codes, norms, outv, n, cfg), 5, 1)
    nb = n * per_vector_bytes(d, 3)
    out["cfg5_V_tq_d128_b3_full_decode"] = {"gbps": round(nb / ms / 1e6, 1), "ms": round(ms, 4),
                                            "pct_peak": round(nb / ms / 1e6 / PEAK_GBPS * 100, 1)}
    del outv, codes, norms
    # keys: KIVI b=4 G=64, full decode
    ccfg = P.ChannelQuantConfig(d, 4, 64)
    nt = L * H * T
    kc = torch.empty(nt * ccfg.codeStride, dtype=torch.uint8, device=dev)
    kr = torch.empty(ccfg.groupCount(nt) * 2 * d, dtype=torch.float16, device=dev)
    for layer in range(L):
        k = biased_keys(torch, gen, dev, H, T, d).reshape(-1, d)
        q.enqueuePerChannelEncode(k, kc, kr, H * T, ccfg, codesOffset=layer * H * T * ccfg.codeStride,
                                  rangesOffset=layer * (H * T // 64) * ccfg.rangeStride)
        del k
    outk = torch.empty((nt, d), dtype=torch.float32, device=dev)
    ms = timer.time(lambda i: q.enqueuePerChannelDecode(kc, kr, outk, nt, ccfg), 5, 1)
    kb = kivi_bytes(nt, d, 4, 64)
    out["cfg5_K_kivi_d128_b4_full_decode"] = {"gbps": round(kb / ms / 1e6, 1), "ms": round(ms, 4),
                                              "pct_peak": round(kb / ms / 1e6 / PEAK_GBPS * 100, 1)}
    del outk, kc, kr
    # d=1024 sweep over 2^20 N(0,1) vectors
    x = torch.randn((1 << 20, 1024), generator=gen, device=dev)
    for b in (2, 3, 4, 8):
        cfgx = P.QuantConfig("turboQuant", 1024, b)
        c = torch.empty((1 << 20) * cfgx.codeStride, dtype=torch.uint8, device=dev)
        s_ = torch.empty(1 << 20, dtype=torch.float32, device=dev)
        o = torch.empty_like(x)
        ms_e = timer.time(lambda i: q.enqueueEncode(x, c, s_, 1 << 20, cfgx), 5, 1)
        ms_d = timer.time(lambda i: q.enqueueDecode(c, s_, o, 1 << 20, cfgx), 5, 1)
        nb = (1 << 20) * per_vector_bytes(1024, b)
        out[f"cfg5_sweep_tq_d1024_b{b}"] = {"encode_gbps": round(nb / ms_e / 1e6, 1),
                                            "decode_gbps": round(nb / ms_d / 1e6, 1)}
        del c, s_, o
    return out


if __name__ == "__main__":
    sys.exit(main())
