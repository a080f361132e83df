#!/usr/bin/env python3
"""Benchmark of the MI355X KV-cache codec. Headline: BASELINE config 5, the largest single-GPU configuration.

    python bench.py [--steps K] [--warmup W] [--extras] [--full] [--sweep CSV] [--sweep-channel CSV] [--no-cpu]
                    [--copy-calib]

A step is one full-cache decode of the Llama-3-8B long-context value cache of config 5: 32 layers x 8 KV heads x
131072 tokens x d = 128 = 33,554,432 vectors (2^32 floats), TurboQuant b = 3, Student-t (nu = 5) values, in ONE
call, with codes, norms and the 17.2 GB fp32 output resident in HBM. value = algorithmic bytes per step / time per
step, algorithmic bytes n (4d + codeStride + 4) = 18.92 GB. The timed region is K back-to-back calls on the codec's
stream between two HIP events on that stream, bracketed by device synchronisations; before it come W warm-up calls
and at least 0.25 s of calls.

Before timing, the encode of the same cache (one call) is checked against the CPU oracle on sampled rows (codes may
differ only at near-boundary coordinates, scales within one float32 ulp), and after it the timed decode output is
checked on the same rows (relative L2 <= 1e-5); the benchmark refuses to report otherwise. Beside it, at the same
footprint: a plain device copy and a plain fill (the second denominator: the box's own streaming bandwidth), the
config-5 key cache (KIVI b = 4, G = 64, one call of 33.5M tokens), per-token append latencies, and the oracle's
CPU decode on a 2^16-vector subset (1 thread), extrapolated per vector.

After config 5, every other row of the north-star target (bulk encode and full-cache decode of every method at
d = 64 and 128), each with its parity gate: config 2 (TurboQuant b = 2, 3, 4 and PolarQuant b = 4 at d = 64, and the
per-step append), config 3 (KIVI d = 64) and config 4 (TurboQuant and PolarQuant at d = 128); `north_star_target`
lists each row's % of peak beside the 70 % target (--no-rows skips them).

--extras adds BASELINE config 1, the encoder-shaped stream ceilings and CPU baselines of configs 2-4, single-call
latency percentiles, float16/bfloat16 caches, decode-step attention over compressed caches and key-bias removal;
--full adds the d = 1024 TurboQuant sweep of config 5; --sweep CSV runs the reference's per-call throughput sweep
(both methods, b = 2 / 4 / 8, d = 64 ... 1024, batches of 1 ... 4096 vectors, the GPU-resident and the array API) and
writes it with the reference's results/throughput.csv columns; --sweep-channel CSV runs its per-channel sweep (KIVI
and TurboQuant on the same keys, b = 2 / 4 / 8, d = 64 ... 1024, 64 / 256 / 4096 tokens) with the columns of its
results/per_channel_throughput.csv.
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
WARMUP_S = 0.25  # minimum warm-up per timed measurement, as the reference's benchmarks (BenchmarkSuite.swift:150-185)
C5 = dict(layers=32, heads=8, tokens=131072, dim=128)
HEADLINE_KERNEL = "pitch::vec_decode<128, 3, false, 0, false>"
HEADLINE_PROFILE = "profiles/vec_decode_d128_b3_config5.md"


def code_stride(d: int, b: int) -> int:
    return ((d * b + 31) // 32) * 4


def per_vector_bytes(d: int, b: int) -> int:
    return 4 * d + code_stride(d, b) + 4


def per_vector_bytes16(d: int, b: int) -> int:
    """Per-vector algorithmic bytes with float16 / bfloat16 vectors: 2d + codeStride + 4."""
    return 2 * d + code_stride(d, b) + 4


def kivi_bytes(n: int, d: int, b: int, G: int, heads: int = 1, elem: int = 4) -> int:
    """n tokens per head: n*(elem*d + codeStride) + groups * 4d per head (elem = bytes per key element)."""
    return heads * (n * (elem * d + code_stride(d, b)) + ((n + G - 1) // G) * 4 * d)


class Timer:
    """HIP events on the stream the codec launches on (torch's current stream, which the codec uses by default)."""

    def __init__(self, torch):
        self.torch = torch
        self.stream = torch.cuda.current_stream()

    def time(self, fn, steps: int, warmup: int) -> float:
        """Average milliseconds per call of fn(i) over `steps` back-to-back calls. Before them: at least `warmup`
        calls and at least WARMUP_S seconds of calls (the GPU's clocks take milliseconds to ramp up), then a device
        synchronisation, then one more untimed call so that the start event is recorded behind queued work rather
        than on an idle queue (whose first launch would add its start-up latency to the timed region)."""
        torch = self.torch
        i, t0 = 0, time.perf_counter()
        while i < warmup or time.perf_counter() - t0 < WARMUP_S:
            fn(i)
            i += 1
            if i % 16 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        fn(i)
        i += 1
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(self.stream)
        for k in range(steps):
            fn(i + k)
        end.record(self.stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps

    def single_calls(self, fn, calls: int = 100) -> dict:
        """The reference's single-call protocol (BenchmarkSuite.swift:161-172): `calls` calls, each alone on the
        stream, timed by HIP events around it and by the host clock around launch + synchronisation; median, p10
        and p90 in microseconds."""
        import numpy as np
        torch = self.torch
        i, t0 = 0, time.perf_counter()
        while i < 10 or time.perf_counter() - t0 < WARMUP_S:
            fn(i)
            i += 1
        torch.cuda.synchronize()
        gpu, wall = [], []
        for k in range(calls):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            w0 = time.perf_counter()
            a.record(self.stream)
            fn(i + k)
            b.record(self.stream)
            b.synchronize()
            wall.append((time.perf_counter() - w0) * 1e6)
            gpu.append(a.elapsed_time(b) * 1e3)

        def pct(v):
            return {"median": round(float(np.median(v)), 2), "p10": round(float(np.percentile(v, 10)), 2),
                    "p90": round(float(np.percentile(v, 90)), 2)}
        return {"gpu_us": pct(gpu), "wall_us": pct(wall)}


def profile_field(rel: str, key: str):
    """A `key: value` line of a committed rocprofv3 summary under profiles/, or None."""
    f = ROOT / rel
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith(key + ":"):
            v = line.split(":", 1)[1].strip()
            try:
                return int(v)
            except ValueError:
                return float(v)
    return None


def sample_rows(n: int, seed: int, extra: int = 1024):
    import numpy as np
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([np.arange(min(64, n)), np.arange(max(0, n - 64), n), rng.integers(0, n, extra)]))


def check_vector_encode(O, method: str, X, C: bytes, S, d: int, b: int, label: str) -> int:
    """Sampled rows of an encode against the oracle: codes equal except at near-boundary coordinates, scales within
    one float32 ulp. Returns the count of (near-boundary) code differences."""
    import numpy as np
    X64 = X.astype(np.float64)
    codes, scales = O.ENCODERS[method](X64, b)
    ours = O.unpack_codes(C, X.shape[0], d, b)
    diff = ours != codes
    if diff.any():
        band = (O.turbo_near_boundary(O.turbo_rotated(X64), b) if method == "turboQuant"
                else O.polar_near_boundary(X64, b))
        if (diff & ~band).any():
            raise SystemExit(f"parity gate failed for {label}: {int((diff & ~band).sum())} codes differ")
    ulps = np.abs(np.asarray(S, np.float32).view(np.int32).astype(np.int64)
                  - np.asarray(scales, np.float32).view(np.int32).astype(np.int64))
    if ulps.max() > 1:
        raise SystemExit(f"parity gate failed for {label}: scales differ by {int(ulps.max())} ulp")
    return int(diff.sum())


def check_vector_decode(O, method: str, C: bytes, S, got, d: int, b: int, label: str) -> float:
    """Sampled rows of a decode against the oracle's decode of the same codes: relative L2 <= 1e-5."""
    import numpy as np
    ref = O.DECODERS[method](O.unpack_codes(C, len(S), d, b), np.asarray(S, np.float64), b)
    got = np.asarray(got, np.float64)
    rel = float(np.max(np.sqrt(((got - ref) ** 2).sum(1) / np.maximum((ref ** 2).sum(1), 1e-300))))
    if rel > 1e-5:
        raise SystemExit(f"decode parity failed for {label}: max rel L2 {rel}")
    return rel


def time_copy_fill(torch, timer, src, dst, steps: int = 10) -> dict:
    """The box's own streaming rates at a given footprint: a device copy src -> dst (bytes read + written) and a
    fill of dst (bytes written), torch's own kernels, timed like the codec."""
    nb = dst.numel() * dst.element_size()
    ms_copy = timer.time(lambda i: dst.copy_(src), steps, 2)
    ms_fill = timer.time(lambda i: dst.fill_(float(i % 7)), steps, 2)
    return {"bytes": nb, "copy_gbps": round(2 * nb / ms_copy / 1e6, 1), "copy_ms": round(ms_copy, 4),
            "fill_gbps": round(nb / ms_fill / 1e6, 1), "fill_ms": round(ms_fill, 4)}


class StreamCeiling:
    """An encoder's bytes with no arithmetic: libpitch_calib.so's pitch_calib_stream reads unit_bytes and writes
    out_words 4-byte words per unit (vector or key row), with its loads in a chosen access shape (the contiguous
    piece of a unit that one load instruction reads, the grid, cached or non-temporal). Timed like the codec on
    the same buffers, it gives the rate any kernel moving those bytes in that shape reaches on this box: the
    shape the encoder uses, and the best of a small sweep of shapes."""

    def __init__(self, torch):
        import ctypes
        self.torch = torch
        lib = ctypes.CDLL(str(ROOT / "pitch_amd" / "libpitch_calib.so"))
        fn = lib.pitch_calib_stream
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                       ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        self.fn = fn
        st = lib.pitch_calib_stream_store
        st.restype = ctypes.c_int
        st.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                       ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        self.store_fn = st
        self.cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count

    def _call(self, src, dst, units: int, unit_bytes: int, out_words: int, seg: int, wgs: int, nt: int) -> None:
        if dst.numel() * dst.element_size() < units * out_words * 4 or src.numel() * src.element_size() < units * unit_bytes:
            raise ValueError("calibration buffers are smaller than the stream")
        rc = self.fn(src.data_ptr(), dst.data_ptr(), units, unit_bytes, out_words, seg, wgs, nt,
                     self.torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError("pitch_calib_stream rejected its arguments")

    def measure_decoder(self, timer, src, dst, units: int, unit_bytes: int, in_words: int, dec_seg: int,
                        dec_mode: int, dec_gbps: float, steps: int, warm: int) -> dict:
        """The decoders' mirror image (pitch_calib_stream_store): in_words words read (coalesced) and unit_bytes
        written per unit, in store pieces of 64-512 bytes, as one persistent launch, one launch of one block per
        workgroup, or launches of one round of 8 workgroups per CU (the config-5 decoders' shape); non-temporal or
        cached stores. dec_seg, dec_mode: the decoder's store piece and grid (0, 1, 2 as above)."""
        if (dst.numel() * dst.element_size() < units * unit_bytes or src.numel() * src.element_size() < units * in_words * 4):
            raise ValueError("calibration buffers are smaller than the stream")
        nbytes = units * (unit_bytes + 4 * in_words)
        wgs = 8 * self.cus
        names = {0: "persistent", 1: "oneblock", 2: "rounds"}
        rates = {}
        stream = self.torch.cuda.current_stream().cuda_stream

        def call(seg, mode, nt):
            if self.store_fn(src.data_ptr(), dst.data_ptr(), units, unit_bytes, in_words, seg, mode, wgs, nt, stream):
                raise RuntimeError("pitch_calib_stream_store rejected its arguments")

        for seg in (64, 128, 256, 512):
            if unit_bytes % seg or unit_bytes // seg > 8:
                continue
            for mode in (0, 1, 2):
                for nt in (1, 0):
                    ms = timer.time(lambda i: call(seg, mode, nt), steps, warm)
                    rates[(seg, mode, nt)] = nbytes / ms / 1e6
        shape = rates[(dec_seg, dec_mode, 1)]
        best = max(rates, key=rates.get)
        return {"bytes_per_call": nbytes,
                "decoder_shape": {"store_piece_bytes": dec_seg, "grid": names[dec_mode], "nontemporal": True,
                                  "gbps": round(shape, 1)},
                "best": {"store_piece_bytes": best[0], "grid": names[best[1]], "nontemporal": bool(best[2]),
                         "gbps": round(rates[best], 1), "pct_peak": round(rates[best] / PEAK_GBPS * 100, 1)},
                "decoder_frac_of_decoder_shape": round(dec_gbps / shape, 3),
                "decoder_frac_of_best": round(dec_gbps / rates[best], 3),
                "all_gbps": {f"piece{k[0]}_{names[k[1]]}_{'nt' if k[2] else 'cached'}": round(v, 1)
                             for k, v in sorted(rates.items())}}

    def measure(self, timer, pairs, units: int, unit_bytes: int, out_words: int, enc_seg: int, enc_gbps: float,
                steps: int, warm: int) -> dict:
        """pairs: (input, output) buffer sets rotated like the encoder's timing. enc_seg: the encoder's load
        piece; the encoder's grid is 3 workgroups per CU, persistent, non-temporal."""
        nbytes = units * (unit_bytes + 4 * out_words)
        rates = {}
        for seg in (64, 128, 256, 512):
            if unit_bytes % seg or unit_bytes // seg > 8:
                continue
            for wgs in (3 * self.cus, 0):
                for nt in (1, 0):
                    ms = timer.time(lambda i: self._call(pairs[i % len(pairs)][0], pairs[i % len(pairs)][1], units,
                                                         unit_bytes, out_words, seg, wgs, nt), steps, warm)
                    rates[(seg, wgs, nt)] = nbytes / ms / 1e6
        enc_shape = rates[(enc_seg, 3 * self.cus, 1)]
        best = max(rates, key=rates.get)
        return {"bytes_per_call": nbytes,
                "encoder_shape": {"load_piece_bytes": enc_seg, "grid": "persistent, 3 workgroups per CU",
                                  "nontemporal": True, "gbps": round(enc_shape, 1)},
                "best": {"load_piece_bytes": best[0],
                         "grid": "persistent, 3 workgroups per CU" if best[1] else "one block per workgroup",
                         "nontemporal": bool(best[2]), "gbps": round(rates[best], 1),
                         "pct_peak": round(rates[best] / PEAK_GBPS * 100, 1)},
                "encoder_frac_of_encoder_shape": round(enc_gbps / enc_shape, 3),
                "encoder_frac_of_best": round(enc_gbps / rates[best], 3),
                "all_gbps": {f"piece{k[0]}_{'persistent' if k[1] else 'oneblock'}_{'nt' if k[2] else 'cached'}":
                             round(v, 1) for k, v in sorted(rates.items())}}


def cpu_time(fn, seconds: float) -> tuple[float, int]:
    """Median seconds of fn() over runs for at least `seconds` (3 warm-ups first, at least 5 runs)."""
    for _ in range(3):
        fn()
    times, t0 = [], time.perf_counter()
    while time.perf_counter() - t0 < seconds or len(times) < 5:
        t1 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t1)
    return sorted(times)[len(times) // 2], len(times)


def host_cpus() -> dict:
    return {"affinity": len(os.sched_getaffinity(0)), "cpu_count": os.cpu_count()}


def cpu_baseline_vector_decode(O, C: bytes, S, d: int, b: int, label: str, seconds: float = 12.0) -> dict:
    """The oracle's decode (numpy, float64 spec semantics, 1 thread) of the sampled vectors, per vector."""
    import numpy as np
    n = len(S)
    codes = O.unpack_codes(C, n, d, b)
    s64 = np.asarray(S, np.float64)
    t, runs = cpu_time(lambda: O.turbo_decode(codes, s64, b), seconds)
    return {"value": round(n * per_vector_bytes(d, b) / t / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle/pitch_oracle.py turbo_decode (float64 numpy, 1 thread) of {n} vectors of the {label} "
                      f"(d={d} b={b}), median of {runs} runs: {t * 1e3:.1f} ms; extrapolated per vector: "
                      f"{n / t:.3e} vectors/s",
            "vectors_per_s": round(n / t, 1), "host_cpus": host_cpus()}


def run_config5_values(torch, q, P, O, W, timer, dev, args) -> tuple[dict, dict]:
    """Config 5 V: generate, encode in one call (checked), copy/fill calibration, timed full-cache decode (checked)."""
    L, H, T, d, b = C5["layers"], C5["heads"], C5["tokens"], C5["dim"], 3
    n = L * H * T
    print(f"# config 5 V: generating {n} Student-t vectors (d={d})", file=sys.stderr, flush=True)
    gen = torch.Generator(device=dev).manual_seed(5)
    x = W.config5_values(torch, gen, dev, L, H, T, d)
    cfg = P.QuantConfig("turboQuant", d, b)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    scales = torch.empty(n, dtype=torch.float32, device=dev)
    print("# config 5 V: encode (one call) + parity gate", file=sys.stderr, flush=True)
    q.enqueueEncode(x, codes, scales, n, cfg)
    torch.cuda.synchronize()
    idx = sample_rows(n, 50)
    it = torch.from_numpy(idx).to(dev)
    X = x[it].cpu().numpy()
    C = codes.view(n, cfg.codeStride)[it].cpu().numpy().tobytes()
    S = scales[it].cpu().numpy()
    diffs = check_vector_encode(O, "turboQuant", X, C, S, d, b, "config 5 V encode")
    ms_enc = timer.time(lambda i: q.enqueueEncode(x, codes, scales, n, cfg), 10, 2)
    out = torch.empty((n, d), dtype=torch.float32, device=dev)
    print("# config 5 V: copy / fill calibration at the same footprint", file=sys.stderr, flush=True)
    calib = time_copy_fill(torch, timer, x, out)
    print("# config 5 V: encoder-shaped stream calibration at the same footprint", file=sys.stderr, flush=True)
    enc_ceiling = StreamCeiling(torch).measure(timer, [(x, out)], n, 4 * d, (cfg.codeStride + 4) // 4, 128,
                                               n * per_vector_bytes(d, b) / ms_enc / 1e6, 3, 1)
    del x
    torch.cuda.empty_cache()
    print("# config 5 V: timing full-cache decode", file=sys.stderr, flush=True)
    ms = timer.time(lambda i: q.enqueueDecode(codes, scales, out, n, cfg), args.steps, args.warmup)
    rel = check_vector_decode(O, "turboQuant", C, S, out[it].cpu().numpy(), d, b, "config 5 V decode")
    nbytes = n * per_vector_bytes(d, b)
    gbps = nbytes / (ms * 1e-3) / 1e9
    print("# config 5 V: decoder-shaped stream calibration at the same footprint", file=sys.stderr, flush=True)
    src = torch.empty(n * ((cfg.codeStride + 4) // 4), dtype=torch.int32, device=dev)
    # the decoder stages a wave's vectors in LDS and writes them whole (each store instruction 1 KB: two 512-byte
    # vectors), one workgroup per block in one launch
    dec_ceiling = StreamCeiling(torch).measure_decoder(timer, src, out, n, 4 * d, (cfg.codeStride + 4) // 4, 512, 1,
                                                       gbps, 3, 1)
    del src
    cpu = None if args.no_cpu else cpu_baseline_vector_decode(
        O, codes[:65536 * cfg.codeStride].cpu().numpy().tobytes(), scales[:65536].cpu().numpy(), d, b,
        "config 5 value cache (first 2^16 vectors)")
    traffic = profile_field(HEADLINE_PROFILE, "traffic_bytes_per_call")
    head = {
        "metric": METRIC, "value": round(gbps, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: Student-t(nu=5) values generated on device (seeded), encoded by the library",
        "config": {"workload": "config 5 V full-cache decode: Llama-3-8B long context, TurboQuant b=3, 32 layers x "
                               "8 KV heads x 131072 tokens x d=128 = 33,554,432 vectors (18.92 GB algorithmic) in "
                               "one call, fp32 output",
                   "method": "turboQuant", "dim": d, "bits": b, "vectors": n, "bytes_per_step": nbytes},
        "vectors_per_s": round(n / (ms * 1e-3), 1),
        "pct_of_hbm_peak": round(100 * gbps / PEAK_GBPS, 2),
        # one call is the kernel's launches over the whole cache: achieved = algorithmic bytes per call / HIP-event
        # time per call (launch gaps included); the rocprofv3 per-launch mean and launch count are from the profile
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / PEAK_GBPS, 4), "traffic": traffic, "kernel": HEADLINE_KERNEL,
                     "step_us_hip_events": round(ms * 1e3, 2),
                     "launches_per_call_rocprof": profile_field(HEADLINE_PROFILE, "launches_per_call"),
                     "kernel_mean_us_per_launch_rocprof": profile_field(HEADLINE_PROFILE, "kernel_mean_us"),
                     "kernel_us_per_call_rocprof": profile_field(HEADLINE_PROFILE, "kernel_us_per_call"),
                     "algorithmic_bytes_per_call": nbytes,
                     "frac_of_measured_fill": round(gbps / calib["fill_gbps"], 4),
                     "frac_of_measured_copy": round(gbps / calib["copy_gbps"], 4),
                     "profile": HEADLINE_PROFILE if traffic else None},
        "parity": {"sampled_rows": int(len(idx)), "encode_code_diffs_near_boundary": diffs,
                   "decode_max_rel_l2": rel},
        "same_footprint_streaming": calib,
        "decode_stream_ceiling": dec_ceiling,
    }
    if cpu:
        head["cpu_baseline"] = cpu
    extra = {"cfg5_V_tq_d128_b3_encode_one_call": {"ms": round(ms_enc, 4),
                                                   "gbps": round(nbytes / ms_enc / 1e6, 1),
                                                   "pct_peak": round(nbytes / ms_enc / 1e6 / PEAK_GBPS * 100, 1),
                                                   "stream_ceiling": enc_ceiling}}
    # per-token append: 8 vectors per layer at codesOffset = (t * 8) * codeStride within each layer's slice
    per_layer = H * T
    xa = torch.randn(L, H, d, device=dev)
    cs = cfg.codeStride

    def append_token(i):
        t = i % T
        for layer in range(L):
            v0 = layer * per_layer + t * H
            q.enqueueEncode(xa[layer], codes, scales, H, cfg, codesOffset=v0 * cs, scalesOffset=v0 * 4)

    ms_tok = timer.time(append_token, 50, 5)
    single = timer.single_calls(lambda i: q.enqueueEncode(xa[i % L], codes, scales, H, cfg,
                                                          codesOffset=((i % L) * per_layer + (i % T) * H) * cs,
                                                          scalesOffset=((i % L) * per_layer + (i % T) * H) * 4))
    # the same append as one batched call over the 32 layers (EncodeBatch -> pitch_enqueue_encode_batch)
    import numpy as np
    tab = P.EncodeBatch(q, cfg, [xa[layer] for layer in range(L)], [codes] * L, [scales] * L)
    lbase = np.arange(L, dtype=np.int64) * per_layer

    def append_token_batched(i):
        v0 = lbase + (i % T) * H
        tab.enqueue(H, codesOffsets=v0 * cs, scalesOffsets=v0 * 4)

    ms_tok_b = timer.time(append_token_batched, 50, 5)
    single_b = timer.single_calls(append_token_batched)
    extra["cfg5_V_append_8_vectors_per_layer"] = {
        "token_all_32_layers_us_backtoback": round(ms_tok * 1e3, 2),
        "per_layer_call_us_backtoback": round(ms_tok * 1e3 / L, 2), "single_call": single,
        "token_all_32_layers_one_batched_call_us_backtoback": round(ms_tok_b * 1e3, 2),
        "batched_single_call": single_b}
    del codes, scales, out, xa
    torch.cuda.empty_cache()
    return head, extra


def run_config5_keys(torch, q, P, O, W, timer, dev, args) -> dict:
    """Config 5 K: KIVI b=4 G=64 over the whole key cache, encode and timed decode in one call each (checked)."""
    import numpy as np
    L, H, T, d, b, G = C5["layers"], C5["heads"], C5["tokens"], C5["dim"], 4, 64
    n = L * H * T
    print(f"# config 5 K: generating {n} keys", file=sys.stderr, flush=True)
    gen = torch.Generator(device=dev).manual_seed(6)
    x = W.config5_keys(torch, gen, dev, L, H, T, d)
    cfg = P.ChannelQuantConfig(d, b, G)
    groups = cfg.groupCount(n)
    codes = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    ranges = torch.empty(groups * 2 * d, dtype=torch.float16, device=dev)
    q.enqueuePerChannelEncode(x, codes, ranges, n, cfg)
    ms_enc = timer.time(lambda i: q.enqueuePerChannelEncode(x, codes, ranges, n, cfg), 3, 1)
    torch.cuda.synchronize()
    picks = sorted({0, groups - 1} | {int(g) for g in np.random.default_rng(60).integers(0, groups, 32)})
    xs = {g: x[g * G:(g + 1) * G].cpu().numpy() for g in picks}
    del x
    torch.cuda.empty_cache()
    out = torch.empty((n, d), dtype=torch.float32, device=dev)
    print("# config 5 K: timing full-cache decode", file=sys.stderr, flush=True)
    ms = timer.time(lambda i: q.enqueuePerChannelDecode(codes, ranges, out, n, cfg), max(5, args.steps // 2),
                    args.warmup)
    for g in picks:           # codes, ranges and decode bit-exact against the oracle
        rc, rr = O.channel_encode(xs[g], b, G)
        got_c = codes[g * G * cfg.codeStride:(g + 1) * G * cfg.codeStride].cpu().numpy().tobytes()
        got_r = ranges[g * 2 * d:(g + 1) * 2 * d].cpu().numpy().view(np.uint16)
        got_o = out[g * G:(g + 1) * G].cpu().numpy()
        if (got_c != O.pack_codes(rc, b) or not np.array_equal(got_r, rr.view(np.uint16).reshape(-1))
                or not np.array_equal(got_o.view(np.uint32), O.channel_decode(rc, rr, b, G).view(np.uint32))):
            raise SystemExit(f"config 5 K parity failed at group {g}")
    kb = kivi_bytes(n, d, b, G)
    res = {"tokens": n, "algorithmic_bytes": kb, "decode_ms": round(ms, 4), "decode_gbps": round(kb / ms / 1e6, 1),
           "decode_pct_peak": round(kb / ms / 1e6 / PEAK_GBPS * 100, 1), "encode_ms": round(ms_enc, 4),
           "encode_gbps": round(kb / ms_enc / 1e6, 1), "encode_pct_peak": round(kb / ms_enc / 1e6 / PEAK_GBPS * 100, 1),
           "parity_groups_bit_exact": len(picks)}
    # the decoder writes 256-byte row pieces (64 channels of a token) and reads codes plus fp16 ranges:
    # 512 + 64 + 8 bytes per token at d = 128, b = 4, G = 64
    print("# config 5 K: decoder-shaped stream calibration at the same footprint", file=sys.stderr, flush=True)
    src = torch.empty(n * 18, dtype=torch.int32, device=dev)
    res["decode_stream_ceiling"] = StreamCeiling(torch).measure_decoder(timer, src, out, n, 4 * d, 18, 256, 2,
                                                                        kb / ms / 1e6, 3, 1)
    del src
    if not args.no_cpu:
        g0 = 65536 // G
        c0 = codes[:65536 * cfg.codeStride].cpu().numpy().tobytes()
        r0 = ranges[:g0 * 2 * d].cpu().numpy().reshape(g0, 2, d)
        cu = O.unpack_codes(c0, 65536, d, b)
        t, runs = cpu_time(lambda: O.channel_decode(cu, r0, b, G), 8.0)
        nb0 = kivi_bytes(65536, d, b, G)
        res["cpu_baseline"] = {"value": round(nb0 / t / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                               "sample": f"oracle channel_decode of the first 2^16 tokens (1 thread), median of "
                                         f"{runs} runs: {t * 1e3:.1f} ms", "tokens_per_s": round(65536 / t, 1)}
    # append of one completed group of one head: G tokens (PerChannelBenchmark.swift:33-85; README.md:65-76)
    xg = torch.randn(G, d, device=dev)
    single = timer.single_calls(lambda i: q.enqueuePerChannelEncode(
        xg, codes, ranges, G, cfg, codesOffset=(i % groups) * G * cfg.codeStride,
        rangesOffset=(i % groups) * cfg.rangeStride))
    res["append_one_group_64_tokens"] = single
    del codes, ranges, out, xg
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--sets", type=int, default=8, help="buffer sets rotated in the configs 2-3 timings")
    ap.add_argument("--extras", action="store_true")
    ap.add_argument("--full", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-keys", action="store_true", help="skip the config-5 key cache")
    ap.add_argument("--no-rows", action="store_true", help="skip configs 2-4 (the target's d = 64 / 128 rows)")
    ap.add_argument("--sweep", metavar="CSV", help="also run the reference's throughput sweep, writing CSV")
    ap.add_argument("--sweep-channel", metavar="CSV",
                    help="also run the reference's per-channel sweep (KIVI and TurboQuant), writing CSV")
    ap.add_argument("--copy-calib", action="store_true", help="also run a plain 1 GiB device copy (PMC scaling)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: the codec needs no collective, and this build measures one GPU's "
              f"share (got --gpus {args.gpus})", file=sys.stderr)
        return 2

    import torch

    import pitch_amd as P
    from pitch_amd import workloads as W
    from oracle import pitch_oracle as O

    if not torch.cuda.is_available():
        print("no HIP device visible", file=sys.stderr)
        return 1
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    q = P.PITCH(device=dev)
    timer = Timer(torch)

    result, extra = run_config5_values(torch, q, P, O, W, timer, dev, args)
    if not args.no_keys:
        extra["cfg5_K_kivi_d128_b4_G64_one_call"] = run_config5_keys(torch, q, P, O, W, timer, dev, args)
    if not args.no_rows:
        rows = run_target_rows(torch, q, P, O, W, timer, dev, args)
        extra.update(rows)
        result["north_star_target"] = target_summary(rows, result, extra)
    if args.extras or args.full:
        extra.update(run_extras(torch, q, P, O, W, timer, dev, args))
    if args.full:
        extra.update(run_full(torch, q, P, timer, dev))
    if args.sweep:
        extra.update(run_sweep(torch, q, P, timer, dev, args.sweep))
    if args.sweep_channel:
        extra.update(run_channel_sweep(torch, q, P, timer, dev, args.sweep_channel))
    result["extra"] = extra
    if args.copy_calib:
        a = torch.empty(1 << 28, dtype=torch.float32, device=dev)
        bb = torch.empty_like(a)
        for _ in range(3):
            bb.copy_(a)
        torch.cuda.synchronize()
        result["copy_calibration"] = {"bytes_read": a.numel() * 4, "bytes_written": a.numel() * 4, "calls": 3}
    print(json.dumps(result), flush=True)
    return 0


# ------------------------------------------------------------------------------- the target's rows (default run)
def pct(nbytes: int, ms: float) -> float:
    return round(nbytes / ms / 1e6 / PEAK_GBPS * 100, 1)


def codec_row(nbytes: int, n: int, ms_enc: float, ms_dec: float, **parity) -> dict:
    """encode / decode GB/s, % of the 8 TB/s peak, ms and vectors per second of one bulk call each."""
    return {"encode_gbps": round(nbytes / ms_enc / 1e6, 1), "decode_gbps": round(nbytes / ms_dec / 1e6, 1),
            "encode_pct_peak": pct(nbytes, ms_enc), "decode_pct_peak": pct(nbytes, ms_dec),
            "encode_ms": round(ms_enc, 5), "decode_ms": round(ms_dec, 5),
            "vectors_per_s_encode": round(n / ms_enc * 1e3, 1), "vectors_per_s_decode": round(n / ms_dec * 1e3, 1),
            **parity}


def run_target_rows(torch, q, P, O, W, timer, dev, args) -> dict:
    """Every (method, d in {64, 128}, bulk encode / full-cache decode) pair of the north-star target, each in one
    call over a whole cache with its parity gate (BenchmarkSuite.swift:100-141 times the same pairs):
    * config 2 (GPT-2 value cache, 393,216 d = 64 vectors): TurboQuant b = 2, 3, 4 and PolarQuant b = 4, over
      `--sets` rotated buffer sets so that no call finds its inputs in the 256 MB Infinity Cache; the per-step
      append of 12 vectors;
    * config 3 (KIVI d = 64, b = 4, G = 64, 8 heads x 32768 tokens in one call), bit-exact on every head;
    * config 4 (Qwen2.5-1.5B keys, 917,504 d = 128 vectors): TurboQuant and PolarQuant b = 4 on the same tensor.
    With --extras, the encoder-shaped stream ceilings and the CPU baselines of these rows too."""
    import numpy as np
    out = {}
    steps, warm = max(20, args.steps), 5
    gen = torch.Generator(device=dev).manual_seed(2)
    # ---- config 2: GPT-2 value cache, bulk encode and full-cache decode over rotated buffer sets
    d, n = 64, 32768 * 12
    print("# config 2: TurboQuant b = 2, 3, 4 and PolarQuant b = 4 at d = 64", file=sys.stderr, flush=True)
    sets = [W.gpt2_values(torch, gen, dev) for _ in range(args.sets)]
    x = sets[0]
    for method, b in (("turboQuant", 2), ("turboQuant", 3), ("turboQuant", 4), ("polarQuant", 4)):
        cfg = P.QuantConfig(method, d, b)
        bufs = []
        for xs in sets:
            c = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
            nm = torch.empty(n, dtype=torch.float32, device=dev)
            q.enqueueEncode(xs, c, nm, n, cfg)
            bufs.append((xs, c, nm, torch.empty((n, d), dtype=torch.float32, device=dev)))
        ms_enc = timer.time(lambda i: q.enqueueEncode(bufs[i % len(bufs)][0], bufs[i % len(bufs)][1],
                                                      bufs[i % len(bufs)][2], n, cfg), steps, warm)
        ms_dec = timer.time(lambda i: q.enqueueDecode(bufs[i % len(bufs)][1], bufs[i % len(bufs)][2],
                                                      bufs[i % len(bufs)][3], n, cfg), steps, warm)
        idx = sample_rows(n, b, 2048)
        it = torch.from_numpy(idx).to(dev)
        C = bufs[0][1].view(n, cfg.codeStride)[it].cpu().numpy().tobytes()
        S = bufs[0][2][it].cpu().numpy()
        label = f"config 2 {method} b={b}"
        diffs = check_vector_encode(O, method, x.view(n, d)[it].cpu().numpy(), C, S, d, b, label)
        rel = check_vector_decode(O, method, C, S, bufs[0][3][it].cpu().numpy(), d, b, label)
        nb = n * per_vector_bytes(d, b)
        key = f"cfg2_{'tq' if method == 'turboQuant' else 'polar'}_d64_b{b}"
        out[key] = codec_row(nb, n, ms_enc, ms_dec, parity_code_diffs_near_boundary=diffs,
                             parity_decode_max_rel_l2=rel)
        if args.extras and method == "turboQuant" and b == 4:
            pairs = [(bf[0], torch.empty(n * 9, dtype=torch.int32, device=dev)) for bf in bufs]
            out[key]["encode_stream_ceiling"] = StreamCeiling(torch).measure(
                timer, pairs, n, 4 * d, (cfg.codeStride + 4) // 4, 64, nb / ms_enc / 1e6, steps, warm)
            del pairs
            if not args.no_cpu:
                out[key]["cpu_baseline"] = cpu_baseline_vector_decode(
                    O, bufs[0][1][:65536 * cfg.codeStride].cpu().numpy().tobytes(), bufs[0][2][:65536].cpu().numpy(),
                    d, b, "config 2 value cache (first 2^16 vectors)", 6.0)
        del bufs
    del sets
    # append-encode latency: 12 vectors per step at codesOffset = t*12*cs
    cfg = P.QuantConfig("turboQuant", d, 3)
    codes = torch.empty(32768 * 12 * cfg.codeStride, dtype=torch.uint8, device=dev)
    norms = torch.empty(32768 * 12, dtype=torch.float32, device=dev)

    def app(i):
        t = i % 32768
        q.enqueueEncode(x, codes, norms, 12, cfg, inputOffset=t * 12 * d * 4, codesOffset=t * 12 * cfg.codeStride,
                        scalesOffset=t * 12 * 4)

    ms_app = timer.time(app, 500, 50)
    out["cfg2_append_encode_12vec"] = {"gpu_us_per_call_backtoback": round(ms_app * 1e3, 2),
                                       "single_call": timer.single_calls(app)}
    del x, codes, norms
    # ---- config 3: KIVI keys, Llama-3.2-1B shape (8 heads x 32768 tokens x 64), G=64, b=4
    print("# config 3: KIVI d = 64", file=sys.stderr, flush=True)
    keys = W.biased_keys(torch, gen, dev, 8, 32768, 64)
    ccfg = P.ChannelQuantConfig(64, 4, 64)
    nt = 32768
    kbufs = []
    for s in range(args.sets):
        kk = keys if s == 0 else W.biased_keys(torch, gen, dev, 8, 32768, 64, first_head=8 * s)
        c = torch.empty(8 * nt * ccfg.codeStride, dtype=torch.uint8, device=dev)
        r = torch.empty(8 * ccfg.groupCount(nt) * 2 * 64, dtype=torch.float16, device=dev)
        kbufs.append((kk, c, r, torch.empty_like(kk)))
    # one call over all heads: groups never cross a head (32768 % 64 == 0)
    ms_ke = timer.time(lambda i: q.enqueuePerChannelEncode(kbufs[i % len(kbufs)][0], kbufs[i % len(kbufs)][1],
                                                           kbufs[i % len(kbufs)][2], 8 * nt, ccfg), steps, warm)
    ms_kd = timer.time(lambda i: q.enqueuePerChannelDecode(kbufs[i % len(kbufs)][1], kbufs[i % len(kbufs)][2],
                                                           kbufs[i % len(kbufs)][3], 8 * nt, ccfg), steps, warm)
    kb = kivi_bytes(nt, 64, 4, 64, heads=8)
    # parity gate for KIVI: codes, ranges and decode bit-exact on every head
    for h in range(8):
        kh = keys[h].cpu().numpy()
        codes_ref, ranges_ref = O.channel_encode(kh, 4, 64)
        ch = kbufs[0][1][h * nt * ccfg.codeStride:(h + 1) * nt * ccfg.codeStride].cpu().numpy().tobytes()
        g = ccfg.groupCount(nt)
        rh = kbufs[0][2][h * g * 128:(h + 1) * g * 128].cpu().numpy()
        dh = kbufs[0][3][h].cpu().numpy()
        if (ch != O.pack_codes(codes_ref, 4) or not np.array_equal(rh.view(np.uint16),
                                                                   ranges_ref.reshape(-1).view(np.uint16))
                or not np.array_equal(dh.view(np.uint32),
                                      O.channel_decode(codes_ref, ranges_ref, 4, 64).view(np.uint32))):
            raise SystemExit(f"config 3 KIVI parity failed at head {h}")
    out["cfg3_kivi_d64_b4_G64"] = codec_row(kb, 8 * nt, ms_ke, ms_kd, bit_exact_all_heads=True)
    if args.extras:
        # the KIVI encoder reads 128-byte row pieces (32 channels of one token) and writes codes plus fp16 ranges:
        # 256 + 32 + 4 bytes per token at d = 64, b = 4, G = 64
        pairs = [(kb_[0], torch.empty(8 * nt * 9, dtype=torch.int32, device=dev)) for kb_ in kbufs]
        out["cfg3_kivi_d64_b4_G64"]["encode_stream_ceiling"] = StreamCeiling(torch).measure(
            timer, pairs, 8 * nt, 256, 9, 128, kb / ms_ke / 1e6, steps, warm)
        del pairs
        if not args.no_cpu:
            k0 = keys[0].cpu().numpy()
            t_e, _ = cpu_time(lambda: O.channel_encode(k0, 4, 64), 4.0)
            cr, rr = O.channel_encode(k0, 4, 64)
            t_d, _ = cpu_time(lambda: O.channel_decode(cr, rr, 4, 64), 4.0)
            kb1 = kivi_bytes(nt, 64, 4, 64)
            out["cfg3_kivi_d64_b4_G64"]["cpu_baseline"] = {
                "encode_gbps": round(kb1 / t_e / 1e9, 4), "decode_gbps": round(kb1 / t_d / 1e9, 4), "cores": 1,
                "kind": "port", "sample": f"oracle channel_encode / channel_decode of one head (32768 tokens), "
                                          f"1 thread: {t_e * 1e3:.1f} / {t_d * 1e3:.1f} ms per head"}
    del kbufs, keys
    # ---- config 4: Qwen2.5-1.5B shape d=128, 28 L x 2 h x 16384 tokens, TurboQuant and PolarQuant b=4
    print("# config 4: TurboQuant and PolarQuant b = 4 at d = 128", file=sys.stderr, flush=True)
    n4 = 28 * 2 * 16384
    # two caches (the second a roll of the first), rotated call by call: a call's 0.53 GB never finds the previous
    # call's inputs or outputs in the 256 MB Infinity Cache
    keys4 = torch.cat([W.qwen_keys(torch, gen, dev, 2, 16384, 128, first_head=2 * layer).reshape(-1, 128)
                       for layer in range(28)])
    inputs4 = [keys4, torch.roll(keys4, 4099, 0).contiguous()]
    ceiling4 = None
    for method in ("turboQuant", "polarQuant"):
        cfg4 = P.QuantConfig(method, 128, 4)
        sets4 = [(xk, torch.empty(n4 * cfg4.codeStride, dtype=torch.uint8, device=dev),
                  torch.empty(n4, dtype=torch.float32, device=dev), torch.empty_like(keys4)) for xk in inputs4]
        for xk, c, s_, _ in sets4:
            q.enqueueEncode(xk, c, s_, n4, cfg4)
        ms_e = timer.time(lambda i: q.enqueueEncode(sets4[i % 2][0], sets4[i % 2][1], sets4[i % 2][2], n4, cfg4),
                          steps, warm)
        ms_d = timer.time(lambda i: q.enqueueDecode(sets4[i % 2][1], sets4[i % 2][2], sets4[i % 2][3], n4, cfg4),
                          steps, warm)
        _, c, s_, o = sets4[0]
        idx = sample_rows(n4, 4, 4096)
        it = torch.from_numpy(idx).to(dev)
        C = c.view(n4, cfg4.codeStride)[it].cpu().numpy().tobytes()
        S = s_[it].cpu().numpy()
        X4 = keys4[it].cpu().numpy()
        diffs = check_vector_encode(O, method, X4, C, S, 128, 4, f"config 4 {method}")
        rel = check_vector_decode(O, method, C, S, o[it].cpu().numpy(), 128, 4, f"config 4 {method}")
        nb = n4 * per_vector_bytes(128, 4)
        key = f"cfg4_{'tq' if method == 'turboQuant' else 'polar'}_d128_b4"
        out[key] = codec_row(nb, n4, ms_e, ms_d, parity_code_diffs_near_boundary=diffs, parity_decode_max_rel_l2=rel)
        if args.extras:
            if ceiling4 is None:  # the same bytes for both methods (codeStride 64 at b = 4)
                o4 = torch.empty(n4 * 17, dtype=torch.int32, device=dev)
                ceiling4 = StreamCeiling(torch).measure(timer, [(keys4, o4)], n4, 512, (cfg4.codeStride + 4) // 4,
                                                        128, nb / ms_e / 1e6, steps, warm)
                del o4
                out[key]["encode_stream_ceiling"] = ceiling4
            else:
                enc = nb / ms_e / 1e6
                out[key]["encode_stream_ceiling"] = {
                    "same_as": "cfg4_tq_d128_b4",
                    "encoder_frac_of_encoder_shape": round(enc / ceiling4["encoder_shape"]["gbps"], 3),
                    "encoder_frac_of_best": round(enc / ceiling4["best"]["gbps"], 3)}
            if not args.no_cpu:
                X64 = X4[:4096].astype(np.float64)
                t_e, _ = cpu_time(lambda: O.ENCODERS[method](X64, 4), 3.0)
                cc, ss_ = O.ENCODERS[method](X64, 4)
                t_d, _ = cpu_time(lambda: O.DECODERS[method](cc, np.asarray(ss_, np.float32).astype(np.float64), 4),
                                  3.0)
                out[key]["cpu_baseline"] = {
                    "encode_gbps": round(4096 * per_vector_bytes(128, 4) / t_e / 1e9, 4),
                    "decode_gbps": round(4096 * per_vector_bytes(128, 4) / t_d / 1e9, 4), "cores": 1, "kind": "port",
                    "sample": "oracle encode / decode of 4096 sampled config-4 vectors, 1 thread, extrapolated per "
                              "vector"}
        if method == "turboQuant":
            out["cfg4_layer_calls_tq_d128_b4"] = run_layer_calls(torch, q, P, timer, sets4[0], cfg4, 28, n4 // 28,
                                                                 steps, warm)
        del c, s_, o, sets4
    del keys4, inputs4
    torch.cuda.empty_cache()
    return out


def run_layer_calls(torch, q, P, timer, bufs, cfg, layers: int, per: int, steps: int, warm: int) -> dict:
    """A model's per-layer calls (README.md:65-76: one enqueueEncode / enqueueDecode per layer's cache): `layers`
    caches of `per` vectors, laid out one after another in the buffers, encoded and decoded as one call per layer
    (back to back) and as one batched call over every layer (EncodeBatch / DecodeBatch); the batched calls must write
    the bytes the per-layer calls write."""
    x, codes, scales, o = bufs
    d, cs = cfg.dim, cfg.codeStride
    nb = layers * per * per_vector_bytes(d, cfg.bits)
    xs = [x[l * per:(l + 1) * per] for l in range(layers)]
    cl = [codes[l * per * cs:(l + 1) * per * cs] for l in range(layers)]
    sl = [scales[l * per:(l + 1) * per] for l in range(layers)]
    ol = [o[l * per:(l + 1) * per] for l in range(layers)]

    def enc_layers(i):
        for l in range(layers):
            q.enqueueEncode(xs[l], cl[l], sl[l], per, cfg)

    def dec_layers(i):
        for l in range(layers):
            q.enqueueDecode(cl[l], sl[l], ol[l], per, cfg)

    etab = P.EncodeBatch(q, cfg, xs, cl, sl)
    dtab = P.DecodeBatch(q, cfg, cl, sl, ol)
    ms_e = timer.time(enc_layers, steps, warm)
    ms_d = timer.time(dec_layers, steps, warm)
    ref_c, ref_s, ref_o = codes.clone(), scales.clone(), o.clone()
    ms_eb = timer.time(lambda i: etab.enqueue(per), steps, warm)
    ms_db = timer.time(lambda i: dtab.enqueue(per), steps, warm)
    torch.cuda.synchronize()
    if not (torch.equal(codes, ref_c) and torch.equal(scales.view(torch.int32), ref_s.view(torch.int32))
            and torch.equal(o.view(torch.int32), ref_o.view(torch.int32))):
        raise SystemExit("layer calls: the batched calls wrote other bytes than the per-layer calls")
    return {"layers": layers, "vectors_per_layer": per,
            "encode_per_layer_calls_us": round(ms_e * 1e3, 2), "encode_per_layer_calls_gbps": round(nb / ms_e / 1e6, 1),
            "encode_one_batched_call_us": round(ms_eb * 1e3, 2),
            "encode_one_batched_call_gbps": round(nb / ms_eb / 1e6, 1), "encode_one_batched_call_pct_peak": pct(nb, ms_eb),
            "decode_per_layer_calls_us": round(ms_d * 1e3, 2), "decode_per_layer_calls_gbps": round(nb / ms_d / 1e6, 1),
            "decode_one_batched_call_us": round(ms_db * 1e3, 2),
            "decode_one_batched_call_gbps": round(nb / ms_db / 1e6, 1), "decode_one_batched_call_pct_peak": pct(nb, ms_db),
            "batched_bytes_equal_per_layer_calls": True}


def target_summary(rows: dict, head: dict, extra: dict) -> dict:
    """% of the 8 TB/s peak of every bulk encode and full-cache decode the north-star target names (d = 64 and
    128, every method), beside the target of 70 %."""
    pcts = {}
    for key, r in rows.items():
        if "encode_pct_peak" in r:
            pcts[f"{key}_encode"] = r["encode_pct_peak"]
            pcts[f"{key}_decode"] = r["decode_pct_peak"]
    pcts["cfg5_V_tq_d128_b3_decode"] = head["pct_of_hbm_peak"]
    enc5 = extra.get("cfg5_V_tq_d128_b3_encode_one_call")
    if enc5:
        pcts["cfg5_V_tq_d128_b3_encode"] = enc5["pct_peak"]
    k5 = extra.get("cfg5_K_kivi_d128_b4_G64_one_call")
    if k5:
        pcts["cfg5_K_kivi_d128_b4_encode"] = k5["encode_pct_peak"]
        pcts["cfg5_K_kivi_d128_b4_decode"] = k5["decode_pct_peak"]
    below = sorted(k for k, v in pcts.items() if v < 70.0)
    return {"target_pct": 70.0, "pct_of_peak": pcts, "rows": len(pcts), "rows_at_or_above": len(pcts) - len(below),
            "below": below, "min_pct": min(pcts.values())}



# ------------------------------------------------------------------------------------------- --sweep
SWEEP_COLUMNS = ("method,bits,dim,batch,phase,api,gpu_us_median,gpu_us_p10,gpu_us_p90,wall_us_median,wall_us_p10,"
                 "wall_us_p90,sustained_gpu_us_per_call,sustained_wall_us_per_call,ns_per_vector_sustained_gpu,"
                 "input_gb_per_s_sustained_gpu")
CHANNEL_SWEEP_COLUMNS = ("method,bits,dim,tokens,phase,gpu_us_median,wall_us_median,sustained_gpu_us_per_call,"
                         "sustained_wall_us_per_call,ns_per_token_sustained_gpu")


def sustained_calls(torch, timer, fn) -> tuple:
    """The reference's sustained dispatches (16 calls encoded into one Metal command buffer, PerChannelBenchmark.swift
    :108-117, BenchmarkSuite.swift:174-183): 16 calls captured once into a HIP graph and the graph replayed 20 times
    between two HIP events (GPU time per call, median; the calls run back to back on the GPU as the command buffer's
    dispatches do), and 20 times 16 calls launched from the host between device synchronisations (wall time per
    call, median). Called after Timer.single_calls' warm-up. The enqueue entry points issue only kernel launches, so
    they can be captured."""
    import numpy as np
    graph, stream = torch.cuda.CUDAGraph(), torch.cuda.Stream()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(16):
            fn()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    per = []
    cur = torch.cuda.current_stream()
    for _ in range(20):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(cur)
        graph.replay()
        b.record(cur)
        b.synchronize()
        per.append(a.elapsed_time(b) * 1e-3 / 16)
    wall = []
    for _ in range(20):
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        for _ in range(16):
            fn()
        torch.cuda.synchronize()
        wall.append((time.perf_counter() - w0) / 16)
    return float(np.median(per)), float(np.median(wall))


def run_sweep(torch, q, P, timer, dev, path: str) -> dict:
    """The reference's throughput sweep (BenchmarkSuite.swift:100-141; its results/throughput.csv has the same
    columns): both methods, b in {2, 4, 8}, d in {64 .. 1024}, batch in {1, 16, 256, 4096}; for each, the GPU-resident
    calls (enqueueEncode / enqueueDecode on device buffers) timed one at a time (100 calls: GPU time by HIP events
    around the call, wall time around launch + synchronisation; median, p10, p90) and back to back (sustained_calls:
    16 calls replayed as one HIP graph, as the reference's 16 dispatches in one command buffer, and 16 calls launched
    from the host for the wall time; medians per call), and the array API (encode of a
    host array, decode of a CompressedBatch to a host array: host copies and the wait included; 30 calls, wall
    time). Input GB/s counts the fp32 input bytes, as the reference's does. Writes the CSV to `path`."""
    import numpy as np
    rows = [SWEEP_COLUMNS]
    g = lambda v: f"{v:.6g}"
    pct = lambda v, p: float(np.sort(v)[min(len(v) - 1, int(round((len(v) - 1) * p)))])

    def wall_calls(fn, n=30):
        for _ in range(3):
            fn()
        out = []
        for _ in range(n):
            w0 = time.perf_counter()
            fn()
            out.append(time.perf_counter() - w0)
        return out

    for dim in (64, 128, 256, 512, 1024):
        for batch in (1, 16, 256, 4096):
            x = np.random.default_rng(7).standard_normal((batch, dim)).astype(np.float32)
            xd = torch.from_numpy(x).to(dev)
            out = torch.empty_like(xd)
            nbytes = batch * dim * 4
            for method in ("turboQuant", "polarQuant"):
                for bits in (2, 4, 8):
                    cfg = P.QuantConfig(method, dim, bits)
                    codes = torch.empty(batch * cfg.codeStride, dtype=torch.uint8, device=dev)
                    scales = torch.empty(batch, device=dev)
                    enc = lambda: q.enqueueEncode(xd, codes, scales, batch, cfg)  # noqa: E731
                    dec = lambda: q.enqueueDecode(codes, scales, out, batch, cfg)  # noqa: E731
                    for phase, fn in (("encode", enc), ("decode", dec)):
                        single = timer.single_calls(lambda i: fn())
                        s_gpu, s_wall = sustained_calls(torch, timer, fn)
                        rows.append(",".join([method, str(bits), str(dim), str(batch), phase, "gpu_resident",
                                              g(single["gpu_us"]["median"]), g(single["gpu_us"]["p10"]),
                                              g(single["gpu_us"]["p90"]), g(single["wall_us"]["median"]),
                                              g(single["wall_us"]["p10"]), g(single["wall_us"]["p90"]),
                                              g(s_gpu * 1e6), g(s_wall * 1e6), g(s_gpu * 1e9 / batch),
                                              g(nbytes / s_gpu / 1e9)]))
                    compressed = q.encode(x.reshape(-1), config=cfg)
                    for phase, fn in (("encode", lambda: q.encode(x.reshape(-1), config=cfg)),
                                      ("decode", lambda: q.decode(compressed))):
                        w = np.asarray(wall_calls(fn)) * 1e6
                        rows.append(",".join([method, str(bits), str(dim), str(batch), phase, "array", "", "", "",
                                              g(pct(w, 0.5)), g(pct(w, 0.1)), g(pct(w, 0.9)), "", "", "", ""]))
            print(f"# sweep d={dim} batch={batch} done", file=sys.stderr, flush=True)
    Path(path).write_text("\n".join(rows) + "\n")
    return {"throughput_sweep": {"csv": path, "rows": len(rows) - 1}}


def run_channel_sweep(torch, q, P, timer, dev, path: str) -> dict:
    """The reference's per-channel sweep (PerChannelBenchmark.swift:24-79; its results/per_channel_throughput.csv has
    the same columns): d in {64 .. 1024}, tokens in {64, 256, 4096}, b in {2, 4, 8}, N(0, 1) keys (seed 7); per shape
    and width the per-channel (KIVI, G = 64) encode and decode and the TurboQuant encode and decode of the same keys,
    each timed one call at a time (100 calls; GPU time by HIP events around the call, wall time around launch and
    synchronisation; medians) and back to back (sustained_calls: the reference's 16 sustained dispatches as one
    replayed HIP graph for GPU time, launched from the host for wall time; medians per call). Writes the CSV to
    `path`."""
    import numpy as np
    rows = [CHANNEL_SWEEP_COLUMNS]
    g = lambda v: f"{v:.6g}"  # noqa: E731
    for dim in (64, 128, 256, 512, 1024):
        for tokens in (64, 256, 4096):
            x = torch.from_numpy(np.random.default_rng(7).standard_normal((tokens, dim)).astype(np.float32)).to(dev)
            out = torch.empty_like(x)
            for bits in (2, 4, 8):
                cc = P.ChannelQuantConfig(dim, bits)
                codes = torch.empty(tokens * cc.codeStride, dtype=torch.uint8, device=dev)
                ranges = torch.empty(cc.groupCount(tokens) * cc.rangeStride // 2, dtype=torch.float16, device=dev)
                tc = P.QuantConfig("turboQuant", dim, bits)
                tcodes = torch.empty(tokens * tc.codeStride, dtype=torch.uint8, device=dev)
                tnorms = torch.empty(tokens, device=dev)
                calls = (("perChannel", "encode", lambda: q.enqueuePerChannelEncode(x, codes, ranges, tokens, cc)),
                         ("perChannel", "decode", lambda: q.enqueuePerChannelDecode(codes, ranges, out, tokens, cc)),
                         ("turboQuant", "encode", lambda: q.enqueueEncode(x, tcodes, tnorms, tokens, tc)),
                         ("turboQuant", "decode", lambda: q.enqueueDecode(tcodes, tnorms, out, tokens, tc)))
                for method, phase, fn in calls:
                    single = timer.single_calls(lambda i: fn())
                    s_gpu, s_wall = sustained_calls(torch, timer, fn)
                    rows.append(",".join([method, str(bits), str(dim), str(tokens), phase,
                                          g(single["gpu_us"]["median"]), g(single["wall_us"]["median"]),
                                          g(s_gpu * 1e6), g(s_wall * 1e6), g(s_gpu * 1e9 / tokens)]))
            print(f"# channel sweep d={dim} tokens={tokens} done", file=sys.stderr, flush=True)
    Path(path).write_text("\n".join(rows) + "\n")
    return {"per_channel_sweep": {"csv": path, "rows": len(rows) - 1}}


# ------------------------------------------------------------------------------------------- --extras
def run_extras(torch, q, P, O, W, timer, dev, args) -> dict:
    """BASELINE config 1, single-call latency percentiles, 16-bit caches, attention and key-bias removal."""
    import numpy as np
    out = {}
    steps, warm = max(20, args.steps), 5
    gen = torch.Generator(device=dev).manual_seed(2)
    # ---- config 1: 4096 x 64 N(0,1) (seed 0), rotation seed 1, b = 4: encode then decode, parity and us per call
    X1 = np.random.default_rng(0).standard_normal((4096, 64)).astype(np.float32)
    cfg1 = P.QuantConfig("turboQuant", 64, 4, 1)
    x1 = torch.from_numpy(X1).to(dev)
    c1 = torch.empty(4096 * cfg1.codeStride, dtype=torch.uint8, device=dev)
    s1 = torch.empty(4096, device=dev)
    o1 = torch.empty_like(x1)
    q.enqueueEncode(x1, c1, s1, 4096, cfg1)
    q.enqueueDecode(c1, s1, o1, 4096, cfg1)
    torch.cuda.synchronize()
    codes1, norms1 = O.turbo_encode(X1.astype(np.float64), 4, 1)
    got1 = O.unpack_codes(c1.cpu().numpy().tobytes(), 4096, 64, 4)
    rec1 = O.turbo_decode(got1, s1.cpu().numpy().astype(np.float64), 4, 1)
    rel1 = float(np.max(np.linalg.norm(o1.cpu().numpy() - rec1, axis=1) / np.linalg.norm(rec1, axis=1)))
    enc_b = timer.time(lambda i: q.enqueueEncode(x1, c1, s1, 4096, cfg1), 200, 20)
    dec_b = timer.time(lambda i: q.enqueueDecode(c1, s1, o1, 4096, cfg1), 200, 20)
    out["cfg1_tq_d64_b4_4096"] = {
        "code_diffs": int((got1 != codes1).sum()), "decode_max_rel_l2": rel1,
        "encode_us_backtoback": round(enc_b * 1e3, 2), "decode_us_backtoback": round(dec_b * 1e3, 2),
        "encode_single_call": timer.single_calls(lambda i: q.enqueueEncode(x1, c1, s1, 4096, cfg1)),
        "decode_single_call": timer.single_calls(lambda i: q.enqueueDecode(c1, s1, o1, 4096, cfg1))}
    if not args.no_cpu:
        t_e, _ = cpu_time(lambda: O.turbo_encode(X1.astype(np.float64), 4, 1), 4.0)
        t_d, _ = cpu_time(lambda: O.turbo_decode(codes1, norms1.astype(np.float32).astype(np.float64), 4, 1), 4.0)
        out["cfg1_tq_d64_b4_4096"]["cpu_baseline_1_thread"] = {
            "encode_us": round(t_e * 1e6, 1), "decode_us": round(t_d * 1e6, 1),
            "encode_gbps": round(4096 * per_vector_bytes(64, 4) / t_e / 1e9, 4),
            "decode_gbps": round(4096 * per_vector_bytes(64, 4) / t_d / 1e9, 4), "kind": "port"}
    # ---- single calls (BenchmarkSuite.swift:28-33,161-172): batch {1, 16, 256, 4096} x d {64, 128, 1024}, b = 4
    sc = {}
    for d in (64, 128, 1024):
        cfg = P.QuantConfig("turboQuant", d, 4)
        xs = torch.randn(4096, d, device=dev)
        cs_ = torch.empty(4096 * cfg.codeStride, dtype=torch.uint8, device=dev)
        ss = torch.empty(4096, device=dev)
        os_ = torch.empty_like(xs)
        q.enqueueEncode(xs, cs_, ss, 4096, cfg)
        for nb in (1, 16, 256, 4096):
            sc[f"d{d}_batch{nb}"] = {
                "encode": timer.single_calls(lambda i: q.enqueueEncode(xs, cs_, ss, nb, cfg)),
                "decode": timer.single_calls(lambda i: q.enqueueDecode(cs_, ss, os_, nb, cfg))}
    out["single_call_tq_b4"] = sc
    x2 = W.gpt2_values(torch, gen, dev)
    keys4 = torch.cat([W.qwen_keys(torch, gen, dev, 2, 16384, 128, first_head=2 * layer).reshape(-1, 128)
                       for layer in range(28)])
    out.update(run_io16(torch, q, P, W, timer, gen, dev, args, x2, keys4))
    del x2, keys4
    torch.cuda.empty_cache()
    out.update(run_attention(torch, q, P, O, W, timer, gen, dev, args))
    out.update(run_decode_step(torch, q, P, timer, gen, dev, args))
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


def run_decode_step(torch, q, P, timer, gen, dev, args) -> dict:
    """A decode step of the config-5 model (Llama-3-8B: 32 layers, 8 KV x 4 query heads, d = 128; TurboQuant b = 4
    keys, b = 3 values) over a cache of T tokens: one batched append of the token's keys and one of its values to
    all 32 layers (pitch_enqueue_encode_batch), then the allocation-free attention of every layer. Timed eagerly
    and as a replay of the same step captured in a HIP graph (torch.cuda.graph); the replay's outputs must equal
    the eager ones bit for bit."""
    out = {}
    layers, heads, nq, d = 32, 8, 4, 128
    kcfg, vcfg = P.QuantConfig("turboQuant", d, 4), P.QuantConfig("turboQuant", d, 3)
    steps, warm = max(20, args.steps), 5
    for T in (4096, 32768):
        n = (T + 1) * heads
        caches = []
        for _ in range(layers):
            kc = torch.empty(n * kcfg.codeStride, dtype=torch.uint8, device=dev)
            vc = torch.empty(n * vcfg.codeStride, dtype=torch.uint8, device=dev)
            ks, vs = torch.empty(n, device=dev), torch.empty(n, device=dev)
            x = torch.randn(T * heads, d, generator=gen, device=dev)
            q.enqueueEncode(x, kc, ks, T * heads, kcfg)
            q.enqueueEncode(x, vc, vs, T * heads, vcfg)
            caches.append((kc, ks, vc, vs))
        new_k = [torch.randn(heads, d, generator=gen, device=dev) for _ in range(layers)]
        new_v = [torch.randn(heads, d, generator=gen, device=dev) for _ in range(layers)]
        Q = [torch.randn(heads, nq, d, generator=gen, device=dev) for _ in range(layers)]
        outs = [torch.empty(heads, nq, d, device=dev) for _ in range(layers)]
        tk = P.EncodeBatch(q, kcfg, new_k, [c[0] for c in caches], [c[1] for c in caches])
        tv = P.EncodeBatch(q, vcfg, new_v, [c[2] for c in caches], [c[3] for c in caches])

        def step(i):
            tk.enqueue(heads, codesOffsets=T * heads * kcfg.codeStride, scalesOffsets=T * heads * 4)
            tv.enqueue(heads, codesOffsets=T * heads * vcfg.codeStride, scalesOffsets=T * heads * 4)
            for l in range(layers):
                c = caches[l]
                q.enqueueAttentionDecode(Q[l], c[0], c[1], c[2], c[3], outs[l], T + 1, kcfg, vcfg, qPerKv=nq,
                                         kvHeads=heads, tokenStride=heads, headStride=1, noAlloc=True)

        ms_eager = timer.time(step, steps, warm)
        torch.cuda.synchronize()
        ref = [o.clone() for o in outs]
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
            step(0)
        torch.cuda.synchronize()
        for o in outs:
            o.zero_()
        ms_graph = timer.time(lambda i: graph.replay(), steps, warm)
        torch.cuda.synchronize()
        if not all(torch.equal(a, b) for a, b in zip(outs, ref)):
            raise SystemExit("decode step: the graph replay's attention differs from the eager step")
        wall = []
        for _ in range(20):
            torch.cuda.synchronize()
            w0 = time.perf_counter()
            graph.replay()
            torch.cuda.synchronize()
            wall.append((time.perf_counter() - w0) * 1e6)
        wall.sort()
        out[f"cfg5_decode_step_32_layers_T{T}"] = {
            "layers": layers, "kv_heads": heads, "q_per_kv": nq, "tokens": T + 1,
            "eager_us_per_step_backtoback": round(ms_eager * 1e3, 1),
            "graph_replay_us_per_step_backtoback": round(ms_graph * 1e3, 1),
            "graph_replay_wall_us_median": round(wall[len(wall) // 2], 1)}
        del caches, graph
        torch.cuda.empty_cache()
    return out


def run_attention(torch, q, P, O, W, timer, gen, dev, args) -> dict:
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
    K = W.biased_keys(torch, gen, dev, kv, T, d)
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
    # key-bias removal inside attention: a config-4 layer (Qwen2.5-1.5B: 2 KV heads x 6 query heads, d = 128) of
    # RoPE'd biased keys encoded with the bias removed, token-major cache (pitch_enqueue_attention_decode_key_bias)
    kv, nq, d, T = 2, 6, 128, 16384
    cfg = P.QuantConfig("turboQuant", d, 4)
    n = kv * T
    inv = 1.0 / 1e6 ** (torch.arange(0, d, 2, dtype=torch.float64) / d)
    ang = torch.arange(T, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat([torch.cos(ang)] * 2, 1).float().to(dev).contiguous()
    sin = torch.cat([torch.sin(ang)] * 2, 1).float().to(dev).contiguous()
    bias = (torch.randn(kv, d, generator=gen, device=dev) * 5).contiguous()
    kb = P.KeyBias(bias, cos, sin, firstPosition=0, heads=kv)
    tpos = torch.arange(n, device=dev) // kv
    bb = bias[torch.arange(n, device=dev) % kv]
    K = (torch.randn(n, d, generator=gen, device=dev) + bb * cos[tpos]
         + torch.cat([-bb[:, d // 2:], bb[:, :d // 2]], 1) * sin[tpos]).contiguous()
    V = torch.randn(n, d, generator=gen, device=dev)
    kc = torch.empty(n * cfg.codeStride, dtype=torch.uint8, device=dev)
    vc = torch.empty_like(kc)
    ks, vs = torch.empty(n, device=dev), torch.empty(n, device=dev)
    q.enqueueEncode(K, kc, ks, n, cfg, keyBias=kb)
    q.enqueueEncode(V, vc, vs, n, cfg)
    Q = torch.randn(kv, nq, d, generator=gen, device=dev)
    o = torch.empty(kv, nq, d, device=dev)
    ws = torch.empty(P.attention_workspace_bytes(cfg, cfg, T, nq, kv), dtype=torch.uint8, device=dev)
    ms = timer.time(lambda i: q.enqueueAttentionDecode(Q, kc, ks, vc, vs, o, T, cfg, qPerKv=nq, kvHeads=kv,
                                                       tokenStride=kv, headStride=1, workspace=ws, keyBias=kb),
                    steps, warm)
    o2 = torch.empty_like(o)
    ms_plain = timer.time(lambda i: q.enqueueAttentionDecode(Q, kc, ks, vc, vs, o2, T, cfg, qPerKv=nq, kvHeads=kv,
                                                             tokenStride=kv, headStride=1, workspace=ws),
                          steps, warm)
    Kd = torch.empty(n, d, device=dev)
    Vd = torch.empty(n, d, device=dev)

    def decode_then_attend_bias(i):
        q.enqueueDecode(kc, ks, Kd, n, cfg, keyBias=kb)
        q.enqueueDecode(vc, vs, Vd, n, cfg)
        Kh = Kd.view(T, kv, d).transpose(0, 1).transpose(1, 2).contiguous()
        S = torch.bmm(Q, Kh) / math.sqrt(d)
        return torch.bmm(torch.softmax(S, -1), Vd.view(T, kv, d).transpose(0, 1).contiguous())

    ms_b = timer.time(decode_then_attend_bias, max(5, steps // 4), 2)
    torch.cuda.synchronize()
    ck = O.unpack_codes(kc.cpu().numpy().tobytes(), n, d, 4).reshape(T, kv, d)[:, 0]
    cv = O.unpack_codes(vc.cpu().numpy().tobytes(), n, d, 4).reshape(T, kv, d)[:, 0]
    Ob = O.key_bias_offsets(bias.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), 0, n, kv).reshape(T, kv, d)
    Kr = O.turbo_decode(ck, ks.view(T, kv)[:, 0].cpu().numpy().astype(np.float64), 4) + Ob[:, 0]
    Vr = O.turbo_decode(cv, vs.view(T, kv)[:, 0].cpu().numpy().astype(np.float64), 4)
    ro, _ = O.attend(Q[0].cpu().numpy().astype(np.float64), Kr, Vr, 1 / math.sqrt(d))
    got = o[0].cpu().numpy().astype(np.float64)
    rel = float(max(np.linalg.norm(got[i] - ro[i]) / np.linalg.norm(ro[i]) for i in range(nq)))
    if rel > 1e-5:
        raise SystemExit(f"attention parity failed for key-bias removal: rel L2 {rel}")
    nb = n * 2 * (cfg.codeStride + 4)
    out["cfg4_qwen_layer_attention_key_bias_T16384"] = {
        "kv_heads": kv, "q_per_kv": nq, "dim": d, "tokens": T, "ms": round(ms, 5), "ms_without_key_bias": round(ms_plain, 5),
        "codes_gbps": round(nb / ms / 1e6, 1), "decode_then_attend_ms": round(ms_b, 4),
        "speedup_vs_decode_then_attend": round(ms_b / ms, 2), "parity_max_rel_l2_head0": rel}
    del K, V, kc, vc, ks, vs, Kd, Vd, ws, cos, sin
    torch.cuda.empty_cache()
    return out


def run_io16(torch, q, P, W, timer, gen, dev, args, x, keys4) -> dict:
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
            kk = W.biased_keys(torch, gen, dev, 8, 32768, 64, first_head=8 * s).reshape(nt, 64).to(dt).contiguous()
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
        # a long 16-bit decode (16x config 3's tokens, two buffer sets past the Infinity Cache), which the wave
        # decoder runs with eight channels per lane; gate: equal to the float32 decode rounded to the 16-bit type
        nl = 16 * nt
        long_list = []
        for s in range(2):
            c = torch.empty(nl * ccfg.codeStride, dtype=torch.uint8, device=dev)
            r = torch.empty(ccfg.groupCount(nl) * 2 * 64, dtype=torch.float16, device=dev)
            q.enqueuePerChannelEncode(torch.randn(nl, 64, generator=gen, device=dev) * 3, c, r, nl, ccfg)
            long_list.append((c, r, torch.empty(nl, 64, dtype=dt, device=dev)))
        ms_l = timer.time(lambda i: q.enqueuePerChannelDecode(long_list[i % 2][0], long_list[i % 2][1],
                                                              long_list[i % 2][2], nl, ccfg), steps, warm)
        o32 = torch.empty(nl, 64, dtype=torch.float32, device=dev)
        q.enqueuePerChannelDecode(long_list[0][0], long_list[0][1], o32, nl, ccfg)
        q.enqueuePerChannelDecode(long_list[0][0], long_list[0][1], long_list[0][2], nl, ccfg)
        same = bool(torch.equal(long_list[0][2].view(torch.int16), o32.to(dt).view(torch.int16)))
        kl = kivi_bytes(nl, 64, 4, 64, elem=2)
        out[f"kivi_d64_b4_G64_{nl}_tokens_decode_{io}"] = {
            "decode_gbps": round(kl / ms_l / 1e6, 1), "decode_ms": round(ms_l, 5),
            "decode_pct_peak": round(kl / ms_l / 1e6 / PEAK_GBPS * 100, 1), "equals_rounded_float32_decode": same}
        if not same:
            raise SystemExit(f"16-bit KIVI long decode ({io}) differs from the rounded float32 decode")
        del long_list, o32
    return out


def run_full(torch, q, P, timer, dev) -> dict:
    """Config 5's d=1024 TurboQuant sweep over 2^20 N(0,1) vectors, b = 2, 3, 4, 8."""
    out = {}
    gen = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn((1 << 20, 1024), generator=gen, device=dev)
    for b in (2, 3, 4, 8):
        cfgx = P.QuantConfig("turboQuant", 1024, b)
        c = torch.empty((1 << 20) * cfgx.codeStride, dtype=torch.uint8, device=dev)
        s_ = torch.empty(1 << 20, dtype=torch.float32, device=dev)
        o = torch.empty_like(x)
        ms_e = timer.time(lambda i: q.enqueueEncode(x, c, s_, 1 << 20, cfgx), 10, 2)
        ms_d = timer.time(lambda i: q.enqueueDecode(c, s_, o, 1 << 20, cfgx), 10, 2)
        nb = (1 << 20) * per_vector_bytes(1024, b)
        out[f"cfg5_sweep_tq_d1024_b{b}"] = {"encode_gbps": round(nb / ms_e / 1e6, 1),
                                            "decode_gbps": round(nb / ms_d / 1e6, 1),
                                            "encode_pct_peak": round(nb / ms_e / 1e6 / PEAK_GBPS * 100, 1),
                                            "decode_pct_peak": round(nb / ms_d / 1e6 / PEAK_GBPS * 100, 1)}
        del c, s_, o
    return out


if __name__ == "__main__":
    sys.exit(main())
