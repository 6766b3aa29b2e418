#!/usr/bin/env python3
"""Benchmark of the MI355X codec path on BASELINE config 2 (other configs with --config).

Workload: Mamba d_model=256, 8 layers, d_state=16,
fp32, random-init weights (seed 0); 64 MiB of interleaved float32 records
(4 exponential(0.1) + 4 uniform(-pi, pi) fields, seed 2) split into 1000
chunks of 67,109 bytes, all 1000 chunks in one batch of lanes.

One step = compress the input (resident in HBM) into a compacted payload in
HBM, then decompress that payload back into HBM and check the round trip.
`value` is the compress throughput in input MB/s (10^6 B/s); the decompress
throughput, the compression ratio, the roofline of the dominant kernel and
the CPU baseline are reported in the same JSON line.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "boa-constrictor_amd"))

METRIC = ("compress & decompress input MB/s at d256×8L, 1000 chunks; "
          "compression ratio")
PEAK_TFLOPS = {"fp32": 157.3, "bf16": 2500.0}  # MI355X dense matrix peaks
PEAK_HBM_GBS = 8000.0     # MI355X HBM3E peak
GEMM_KERNEL = {"fp32": "boa::gemm_f32_kernel<128, 256, 4, 4, 16, 0|1|2>",
               "bf16": "boa::gemm_bf16_kernel<256, 256, 4, 4, 64, 1|2, 0|1|2>"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_f32_c2_traffic.json")


def gemm_traffic_bytes():
    """HBM bytes per launch of the dominant GEMM from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs, scaled by the copy-kernel calibration."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return round((t["fetch_kib_per_dispatch"] * t["fetch_scale"] +
                      t["write_kib_per_dispatch"] * t["write_scale"]) * 1024)
    except (OSError, KeyError, ValueError):
        return None


def copy_calibration(nbytes: int, reps: int) -> int:
    """A plain device copy of `nbytes` (torch's copy kernel), for scaling the
    FETCH_SIZE / WRITE_SIZE counters."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": nbytes, "reps": reps}), flush=True)
    return 0


def uvarint_len(x: int) -> int:
    n = 1
    while x >= 0x80:
        x >>= 7
        n += 1
    return n


def container_bytes(stream_bytes, n_chunks) -> int:
    # header 33 + payload + "IDX2" + first bytes + LEB128 lengths + CRC
    return 33 + int(sum(stream_bytes)) + 4 + n_chunks + sum(uvarint_len(int(x)) for x in stream_bytes) + 4


def cpu_baseline(weights, data, chunk, n_chunks, sample_chunks, sample_len, threads, d, L, ds,
                 bf16=False):
    """Time the CPU oracle on the first `sample_chunks` chunks x `sample_len` bytes."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import refcpu
    sample = b"".join(data[c * chunk: c * chunk + sample_len] for c in range(min(sample_chunks, n_chunks)))
    m = refcpu.Model(weights, d, L, ds, bf16=bf16)
    t0 = time.perf_counter()
    blob = m.compress(sample, chunk_size=sample_len, n_threads=threads)
    t1 = time.perf_counter()
    back = m.decompress(blob, n_threads=threads)
    t2 = time.perf_counter()
    m.close()
    assert back == sample, "CPU oracle round trip failed"
    return dict(compress_mb_s=len(sample) / (t1 - t0) / 1e6,
                decompress_mb_s=len(sample) / (t2 - t1) / 1e6,
                bytes=len(sample), compress_s=t1 - t0, decompress_s=t2 - t1,
                blob=blob)


def decode_step_profile(codec, lanes: int, ds: int, d: int, bf16: bool, steps: int = 32) -> dict:
    """Per-class kernel times of `steps` decode steps over `lanes` lanes,
    launched directly (not graph-replayed) with HIP events around every
    kernel; the scan's algorithmic bytes give its HBM roofline."""
    import torch
    tok = torch.randint(0, 256, (lanes,), dtype=torch.uint8, device="cuda")
    logits = torch.empty(lanes, 256, device="cuda")
    codec.reset_state(lanes)
    for _ in range(3):
        codec.step_batch(tok.data_ptr(), lanes, logits.data_ptr())
    torch.cuda.synchronize()
    codec.profile(True)
    codec.profile_reset()
    for _ in range(steps):
        codec.step_batch(tok.data_ptr(), lanes, logits.data_ptr())
    torch.cuda.synchronize()
    p = codec.profile_read()
    codec.profile(False)
    sc = p["scan"]
    gbs = sc["work"] / (sc["ms"] * 1e-3) / 1e9 if sc["ms"] > 0 else 0.0
    di = 2 * d
    return {
        "lanes": lanes, "steps": steps, "launch": "direct (HIP events per kernel)",
        "kernel_us_per_step": {k: round(v["ms"] * 1e3 / steps, 2) for k, v in p.items() if v["ms"] > 0},
        "roofline_scan": {
            "bound": "hbm",
            "kernel": f"boa::{'dec_b16_scan_kernel' if bf16 else 'dec_scan_kernel'}"
                      f"<{ds}, {8 if d <= 128 else (16 if d <= 256 else 32)}, true|false>"
                      " (state cached | streamed, by layer)",
            "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / PEAK_HBM_GBS, 4),
            "avg_launch_us": round(sc["ms"] * 1e3 / max(sc["launches"], 1), 2),
            "bytes_per_launch": round(sc["work"] / max(sc["launches"], 1)),
            "bytes_per_lane_layer": f"8*di*ds + {2 if bf16 else 4}*(3*di + R), di = {di}, ds = {ds}",
        },
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1)
    ap.add_argument("--warmup", type=int, default=0)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                    help="BASELINE config (c2 is the metric's config)")
    ap.add_argument("--chunks", type=int, default=0)
    ap.add_argument("--chunk-len", type=int, default=0,
                    help="probe only: shorten every chunk to this many bytes (not the metric config)")
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-sample-chunks", type=int, default=0)
    ap.add_argument("--cpu-sample-len", type=int, default=4096)
    ap.add_argument("--no-decompress", action="store_true")
    ap.add_argument("--warm-start", type=int, default=0, metavar="B",
                    help="warm-start interleave over B lanes (boa.cpp --warm-start with "
                         "--gpu-batch B); not the metric config")
    ap.add_argument("--host-path", action="store_true",
                    help="also time the host-buffer path (bytes in host memory -> BOA2 container "
                         "in host memory, PCIe transfers included)")
    ap.add_argument("--copy-calibrate", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (counter calibration)")
    args = ap.parse_args()
    if args.copy_calibrate:
        return copy_calibration(args.copy_calibrate, 5)

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by chunk across GPUs; no multi-GPU code is built)",
              file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import boa_hip
    import synth

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    cfg = synth.CONFIGS[args.config]
    d, L, ds, prec = cfg["d_model"], cfg["n_layers"], cfg["d_state"], cfg["precision"]
    tmp = tempfile.mkdtemp(prefix="boa_bench_")
    weights = os.path.join(tmp, f"{args.config}_d{d}_L{L}_seed0.bin")
    synth.write_random_weights(weights, d, L, ds, seed=0)
    data = cfg["gen"]()
    n_chunks = args.chunks or cfg["chunks"]
    chunk = synth.chunk_size_for(len(data), n_chunks)
    workload = args.config
    if args.chunk_len:
        full = chunk
        chunk = args.chunk_len
        data = b"".join(data[c * full: c * full + chunk] for c in range(n_chunks))
        workload = f"{args.config}-probe-{chunk}B-chunks"
    if args.warm_start:
        workload += f"-warm{args.warm_start}"
    n = len(data)
    n_chunks = math.ceil(n / chunk)
    print(f"[bench] {workload}: {n} bytes, {n_chunks} chunks of {chunk} B", file=sys.stderr, flush=True)

    stream = torch.cuda.current_stream()
    codec = boa_hip.Codec(d, L, ds, max_lanes=n_chunks, tile=args.tile, precision=prec)
    codec.set_stream(stream.cuda_stream)
    codec.load_weights(weights)
    d_data = torch.frombuffer(bytearray(data), dtype=torch.uint8).cuda()
    cap = boa_hip.payload_bound_words(n, chunk)
    d_pay = torch.empty(cap, dtype=torch.int32, device="cuda")
    d_out = torch.empty(n, dtype=torch.uint8, device="cuda")

    # load every kernel once (module load, first-touch of buffers)
    prime = min(n, n_chunks * 64)
    codec.compress_device(d_data, prime, 64, d_pay, cap)
    torch.cuda.synchronize()
    codec.set_warm_start(args.warm_start)

    def step(profile: bool):
        torch.cuda.synchronize()
        codec.profile(profile)
        if profile:
            codec.profile_reset()
        t0 = time.perf_counter()
        lens, first, words = codec.compress_device(d_data, n, chunk, d_pay, cap)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        prof = codec.profile_read() if profile else None
        codec.profile(False)
        t_dec = float("nan")
        ok = None
        if not args.no_decompress:
            offs = np.zeros(len(lens), np.uint64)
            offs[1:] = np.cumsum(lens[:-1] // 4)
            last = n - (n_chunks - 1) * chunk
            d_out.zero_()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            codec.decompress_device(d_pay, offs, lens, first, chunk, last, d_out)
            torch.cuda.synchronize()
            t_dec = time.perf_counter() - t2
            ok = bool(torch.equal(d_out, d_data))
        return t1 - t0, t_dec, lens, ok, prof

    for w in range(args.warmup):
        print(f"[bench] warmup step {w}", file=sys.stderr, flush=True)
        step(False)
    t_c = t_d = 0.0
    ok_all = True
    prof = None
    lens = None
    for k in range(args.steps):
        tc, td, lens, ok, p = step(profile=True)
        print(f"[bench] step {k}: compress {tc:.3f} s, decompress {td:.3f} s, round trip {ok}",
              file=sys.stderr, flush=True)
        t_c += tc
        t_d += td
        ok_all = ok_all and (ok is not False)
        prof = p
    K = args.steps
    comp_mb_s = n * K / t_c / 1e6
    dec_mb_s = n * K / t_d / 1e6 if not args.no_decompress else None
    ratio = n / container_bytes(lens, n_chunks)

    # per-class kernel times come from HIP events recorded around every
    # launch on the stream the kernels run on (boa_profile_*)
    g = prof["gemm"]
    gemm_tflops = g["work"] / (g["ms"] * 1e-3) / 1e12 if g["ms"] > 0 else 0.0
    kernel_ms = {k: round(v["ms"], 3) for k, v in prof.items()}
    roofline = {
        "bound": "mfma",
        "kernel": GEMM_KERNEL[prec],
        "achieved": round(gemm_tflops, 2),
        "peak": PEAK_TFLOPS[prec],
        "unit": "TFLOP/s",
        "frac": round(gemm_tflops / PEAK_TFLOPS[prec], 4),
        "traffic": gemm_traffic_bytes() if workload == "c2" else None,
        "launches": g["launches"],
        "avg_launch_ms": round(g["ms"] / max(g["launches"], 1), 4),
        "flop_per_launch": round(g["work"] / max(g["launches"], 1)),
    }
    sc = prof["scan"]
    scan_gbs = sc["work"] / (sc["ms"] * 1e-3) / 1e9 if sc["ms"] > 0 else 0.0
    roofline_scan = {
        "bound": "hbm",
        "kernel": f"boa::scan_chunk_kernel<{ds}, {8 if d <= 128 else (16 if d <= 256 else 32)}>",
        "achieved": round(scan_gbs, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(scan_gbs / PEAK_HBM_GBS, 4),
        "launches": sc["launches"],
        "avg_launch_ms": round(sc["ms"] / max(sc["launches"], 1), 4),
        "bytes_per_launch": round(sc["work"] / max(sc["launches"], 1)),
    }

    cd_ = prof["cdf"]
    cdf_gbs = cd_["work"] / (cd_["ms"] * 1e-3) / 1e9 if cd_["ms"] > 0 else 0.0
    roofline_coder = {
        "bound": "hbm",
        "kernel": "boa::cdf_targets_kernel",
        "achieved": round(cdf_gbs, 1),
        "peak": PEAK_HBM_GBS,
        "unit": "GB/s",
        "frac": round(cdf_gbs / PEAK_HBM_GBS, 4),
        "launches": cd_["launches"],
        "avg_launch_ms": round(cd_["ms"] / max(cd_["launches"], 1), 4),
        "bytes_per_launch": round(cd_["work"] / max(cd_["launches"], 1)),
    }

    # The decode step's kernels, timed with HIP events on a few directly
    # launched steps (boa_step_batch) after the timed region; the decode
    # scan is the step's HBM-bound kernel.
    dec_step = None
    if not args.no_decompress:
        dec_step = decode_step_profile(codec, n_chunks, ds, d, prec == "bf16")

    host = None
    if args.host_path:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        blob = codec.compress(data, chunk_size=chunk)
        t1 = time.perf_counter()
        back = codec.decompress(blob) if not args.no_decompress else data
        t2 = time.perf_counter()
        host = {"compress_mb_s": round(n / (t1 - t0) / 1e6, 4),
                "decompress_mb_s": round(n / (t2 - t1) / 1e6, 4) if not args.no_decompress else None,
                "container_bytes": len(blob), "roundtrip_ok": back == data,
                "container_matches_device_path": len(blob) == container_bytes(lens, n_chunks)}
        ok_all = ok_all and host["roundtrip_ok"]

    cpu = None
    if not args.no_cpu:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        sample_chunks = args.cpu_sample_chunks or 4 * threads
        print(f"[bench] cpu baseline: {sample_chunks} chunks x {args.cpu_sample_len} B on {threads} threads",
              file=sys.stderr, flush=True)
        cb = cpu_baseline(weights, data, chunk, n_chunks, sample_chunks, args.cpu_sample_len,
                          threads, d, L, ds, bf16=prec == "bf16")
        cpu = {"value": round(cb["compress_mb_s"], 5), "unit": "MB/s", "cores": threads,
               "kind": "port",
               "sample": f"first {args.cpu_sample_len} B of each of the first {sample_chunks} chunks "
                         f"({cb['bytes']} B), oracle/refcpu compress (OpenMP over chunks)",
               "decompress_value": round(cb["decompress_mb_s"], 5),
               "compress_s": round(cb["compress_s"], 2), "decompress_s": round(cb["decompress_s"], 2)}

    out = {
        "metric": METRIC,
        "value": round(comp_mb_s, 4),
        "unit": "MB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round((t_c + (0 if args.no_decompress else t_d)) / K * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if prec == "fp32" else "bf16",
        "data": "synthetic",
        "config": {"workload": workload, "d_model": d, "n_layers": L, "d_state": ds,
                   "chunks": n_chunks, "chunk_len": chunk, "input_bytes": n,
                   "precision": prec, "warm_start": args.warm_start,
                   "weights": "random-init seed 0",
                   "input": f"synth.gen_{args.config}"},
        "compress_mb_s": round(comp_mb_s, 4),
        "decompress_mb_s": round(dec_mb_s, 4) if dec_mb_s else None,
        "compression_ratio": round(ratio, 5),
        "roundtrip_ok": ok_all,
        "compress_kernel_ms": kernel_ms,
        "roofline": roofline,
        "roofline_scan": roofline_scan,
        "roofline_coder": roofline_coder,
        "decode_step": dec_step,
        "cpu_baseline": cpu,
    }
    if host:
        out["host_path"] = host
    if cpu:
        out["speedup_vs_cpu_compress"] = round(comp_mb_s / cpu["value"], 1)
    print(json.dumps(out), flush=True)
    codec.close()
    return 0 if ok_all else 1


if __name__ == "__main__":
    sys.exit(main())
