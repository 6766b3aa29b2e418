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

Timing: at most one warmup step (its compress half profiled per kernel with
HIP events), then up to K timed steps without events, as many as fit the
run's wall budget (--budget-s, default 470 s; the line reports the steps
actually timed), then a decode-step kernel profile, one host-buffer round
trip (PCIe-inclusive, reported beside the device-resident `value`) and the
CPU baseline.  Progress goes to stderr at least every 15 s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--budget-s S]
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
DEC_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "dec_ln_gemm_c2_traffic.json")


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


def dec_ln_gemm_traffic_bytes():
    """HBM bytes per launch of the decode LayerNorm GEMMs at the C2 model and
    1000 lanes (in_proj and FF1 launch equally often per step: their mean),
    from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE runs, scaled by the
    copy-kernel calibration."""
    try:
        with open(DEC_TRAFFIC_FILE) as f:
            t = json.load(f)
        ip = t["in_proj_fetch_kib_per_dispatch"] * t["fetch_scale"] + \
            t["in_proj_write_kib_per_dispatch"] * t["write_scale"]
        ff = t["ff1_fetch_kib_per_dispatch"] * t["fetch_scale"] + \
            t["ff1_write_kib_per_dispatch"] * t["write_scale"]
        return round((ip + ff) / 2 * 1024)
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


def decode_steps_only(config: str, steps: int, lanes: int = 0) -> int:
    """Only `steps` directly launched decode steps (boa_step_batch) of the
    config's model (random-init, seed 0) over its lane count: the workload of
    the decode-step counter profiles (rocprofv3 --pmc)."""
    import torch
    import boa_hip
    import synth
    cfg = synth.CONFIGS[config]
    d, L, ds, prec = cfg["d_model"], cfg["n_layers"], cfg["d_state"], cfg["precision"]
    lanes = lanes or cfg["chunks"]
    tmp = tempfile.mkdtemp(prefix="boa_steps_")
    w = os.path.join(tmp, f"{config}.bin")
    synth.write_random_weights(w, d, L, ds, seed=0)
    c = boa_hip.Codec(d, L, ds, max_lanes=lanes, precision=prec)
    c.set_stream(torch.cuda.current_stream().cuda_stream)
    c.load_weights(w)
    c.reset_state(lanes)
    tok = torch.randint(0, 256, (lanes,), dtype=torch.uint8, device="cuda",
                        generator=torch.Generator(device="cuda").manual_seed(0))
    logits = torch.empty(lanes * 256, dtype=torch.float32, device="cuda")
    for _ in range(steps):
        c.step_batch(tok.data_ptr(), lanes, logits.data_ptr())
    torch.cuda.synchronize()
    c.close()
    print(json.dumps({"decode_steps": steps, "config": config, "lanes": lanes,
                      "plan": "boa_step_batch, directly launched"}), flush=True)
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
    """Time the CPU oracle on the first `sample_chunks` chunks x `sample_len`
    bytes, built for x86-64-v4 (AVX-512) where the host has it, else for
    x86-64-v3 (AVX2 + FMA); both builds compute the same bits."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    if "refcpu" not in sys.modules:
        with open("/proc/cpuinfo") as f:
            flags = next((ln.split(":", 1)[1].split() for ln in f if ln.startswith("flags")), [])
        if {"avx512f", "avx512bw", "avx512cd", "avx512dq", "avx512vl"} <= set(flags):
            os.environ["REFCPU_ISA"] = "v4"
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
                blob=blob, isa=refcpu.ISA, lib=os.path.basename(refcpu.LIB_PATH))


def decode_step_profile(codec, lanes: int, steps: int = 32) -> dict:
    """Per-class kernel times of `steps` decode steps over `lanes` lanes,
    launched directly (not graph-replayed) with HIP events around every
    kernel on the launch stream."""
    import torch
    tok = torch.randint(0, 256, (lanes,), dtype=torch.uint8, device="cuda")
    logits = torch.empty(lanes, 256, device="cuda")
    codec.reset_state(lanes)
    for _ in range(3):
        codec.step_batch(tok.data_ptr(), lanes, logits.data_ptr())
    torch.cuda.synchronize()
    codec.profile(True)
    codec.profile_reset()
    # a GPU-side wait first, so that every step is queued before the GPU
    # runs it: the events then time the GPU alone, not host launch gaps
    gpu_hold(torch)
    for _ in range(steps):
        codec.step_batch(tok.data_ptr(), lanes, logits.data_ptr())
    torch.cuda.synchronize()
    p = codec.profile_read()
    codec.profile(False)
    return {k: dict(us_per_step=v["ms"] * 1e3 / steps, launches_per_step=v["launches"] / steps,
                    work_per_step=v["work"] / steps) for k, v in p.items() if v["launches"]}


def decode_coder_profile(codec, torch, data: bytes, chunk: int, n_chunks: int, steps: int = 64):
    """Per-launch time of the decode coder step (the CDF, the symbol search
    and the coder advance; head.2 fused in where the plan fuses it) from a
    profiled decompress of the first `steps` + 1 bytes of every chunk, at the
    config's lane count: one launch per step, HIP events in each dispatch."""
    probe = b"".join(data[c * chunk: c * chunk + steps + 1] for c in range(n_chunks))
    blob = codec.compress(probe, chunk_size=steps + 1)
    torch.cuda.synchronize()
    codec.profile(True)
    codec.profile_reset()
    back = codec.decompress(blob)
    torch.cuda.synchronize()
    p = codec.profile_read()
    codec.profile(False)
    assert back == probe, "decode coder probe round trip failed"
    return p["decode"]


# Compiled VALU instructions per element (token x channel) of the compress
# scan's token loop (scan_chunk_sload_kernel, the large-grid form), counted
# from this build's gfx950 assembly (hipcc --cuda-device-only -S of mamba.hip;
# instructions between the loop header and its back branch, one token per
# iteration): fp32 d_state 16 (the reference's rounding, software exp2) and
# bf16 (hardware exp; the fused update at d_state 16).
SCAN_VALU_PER_ELEMENT = {("fp32", 16): 409, ("fp32", 32): 713, ("bf16", 16): 134, ("bf16", 32): 323}
# MI355X's published fp32 vector peak, 157.3 TFLOP/s, as wave64 FMA
# instructions per second (64 lanes x 2 FLOP): 1,228.8 G/s
VALU_ISSUE_PEAK = 157.3e12 / 128


def gpu_hold(torch, ms: float = 60.0):
    """Queue a GPU-side busy wait of about `ms` on the current stream."""
    torch.cuda._sleep(int(ms * 1e-3 * 2.4e9))


def cpu_info() -> dict:
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "affinity": affinity, "model": model,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def roofline_entry(kernel, bound, achieved, peak, unit, avg_launch, per_launch, per_launch_key,
                   traffic=None, **extra):
    d = {"bound": bound, "kernel": kernel, "achieved": round(achieved, 2), "peak": peak,
         "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
         "avg_launch_us": round(avg_launch, 2), per_launch_key: round(per_launch)}
    d.update(extra)
    return d


def main() -> int:
    t_start = time.perf_counter()
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--budget-s", type=float, default=470.0,
                    help="wall-clock budget of the whole run; timed steps beyond it are skipped "
                         "(the line reports the steps actually timed)")
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"],
                    help="BASELINE config (c2 is the metric's config)")
    ap.add_argument("--chunks", type=int, default=0)
    ap.add_argument("--chunk-len", type=int, default=0,
                    help="probe only: shorten every chunk to this many bytes (not the metric config)")
    ap.add_argument("--tile", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--cpu-sample-chunks", type=int, default=64)
    ap.add_argument("--cpu-sample-len", type=int, default=4096)
    ap.add_argument("--no-decompress", action="store_true")
    ap.add_argument("--no-host-path", action="store_true",
                    help="skip the host-buffer (PCIe-inclusive) round trip")
    ap.add_argument("--warm-start", type=int, default=0, metavar="B",
                    help="warm-start interleave over B lanes (boa.cpp --warm-start with "
                         "--gpu-batch B); not the metric config")
    ap.add_argument("--copy-calibrate", type=int, default=0, metavar="BYTES",
                    help="only run a plain device copy of BYTES (counter calibration)")
    ap.add_argument("--part", default="", metavar="I/N",
                    help="round-trip only part I of N (0-based) of the config's chunks, a "
                         "contiguous share at the config's chunk size; the timed step also "
                         "carries the kernel profile (no second compress pass)")
    ap.add_argument("--decode-steps", type=int, default=0, metavar="N",
                    help="only run N directly launched decode steps of --config over its "
                         "lane count (the workload of the decode counter profiles)")
    args = ap.parse_args()
    if args.copy_calibrate:
        return copy_calibration(args.copy_calibrate, 5)
    if args.decode_steps:
        return decode_steps_only(args.config, args.decode_steps, args.chunks)

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard by chunk across GPUs; no multi-GPU code is built)",
              file=sys.stderr)
        return 2

    def log(msg):
        print(f"[bench {time.perf_counter() - t_start:7.1f}s] {msg}", file=sys.stderr, flush=True)

    import numpy as np
    import torch
    import boa_hip
    import synth

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    log("torch and the codec library loaded")
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
    part = None
    if args.part:
        pi, pn = (int(v) for v in args.part.split("/"))
        total = math.ceil(len(data) / chunk)
        if not 0 <= pi < pn <= total:
            print(f"bench.py: bad --part {args.part} for {total} chunks", file=sys.stderr)
            return 2
        c0, c1 = pi * total // pn, (pi + 1) * total // pn
        data = data[c0 * chunk: c1 * chunk]
        part = {"index": pi, "of": pn, "chunks": [c0, c1], "chunks_total": total}
        workload += f"-part{pi}of{pn}"
    if args.warm_start:
        workload += f"-warm{args.warm_start}"
    n = len(data)
    n_chunks = math.ceil(n / chunk)
    log(f"{workload}: {n} bytes, {n_chunks} chunks of {chunk} B")

    stream = torch.cuda.current_stream()
    codec = boa_hip.Codec(d, L, ds, max_lanes=n_chunks, tile=args.tile, precision=prec)
    codec.set_stream(stream.cuda_stream)
    codec.load_weights(weights)
    d_data = torch.frombuffer(bytearray(data), dtype=torch.uint8).cuda()
    cap = boa_hip.payload_bound_words(n, chunk)
    d_pay = torch.empty(cap, dtype=torch.int32, device="cuda")
    d_out = torch.empty(n, dtype=torch.uint8, device="cuda")

    last_report = [time.perf_counter()]

    def progress(phase, done, total):
        now = time.perf_counter()
        if now - last_report[0] >= 15.0:
            last_report[0] = now
            log(f"  {'compress' if phase == 0 else 'decompress'}: {done / 1e6:.1f} of "
                f"{total / 1e6:.1f} MB")

    codec.set_progress(progress)

    # load every kernel once (module load, first touch of the buffers)
    prime = min(n, n_chunks * 64)
    codec.compress_device(d_data, prime, 64, d_pay, cap)
    torch.cuda.synchronize()
    codec.set_warm_start(args.warm_start)
    last = n - (n_chunks - 1) * chunk

    def step(profile: bool):
        """One pass of the path: compress the HBM-resident input, decompress
        it back, check the round trip.  Returns (compress s, decompress s,
        stream lengths, round trip ok, per-class profile of the compress)."""
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
            d_out.zero_()
            torch.cuda.synchronize()
            t2 = time.perf_counter()
            codec.decompress_device(d_pay, offs, lens, first, chunk, last, d_out)
            torch.cuda.synchronize()
            t_dec = time.perf_counter() - t2
            ok = bool(torch.equal(d_out, d_data))
        return t1 - t0, t_dec, lens, ok, prof

    # Warmup: at most one full step, with per-kernel HIP-event profiling of
    # its compress half (the timed steps run without events).
    prof = None
    warm_done = 0
    step_s = None
    if args.warmup > 0:
        log("warmup step (compress kernels profiled with HIP events)")
        tc, td, lens, ok, prof = step(profile=True)
        warm_done = 1
        step_s = tc + (0 if args.no_decompress else td)
        log(f"warmup: compress {tc:.2f} s, decompress {td:.2f} s, round trip {ok}")
        if ok is False:
            print("bench.py: warmup round trip failed", file=sys.stderr)
            return 1

    # Timed steps, within the run's wall budget: reserve the host-path round
    # trip, the decode-step profile, the CPU baseline and a margin.
    def reserve():
        r = 45.0 + (0 if args.no_cpu else 45.0)
        if not args.no_host_path and step_s:
            r += step_s * 1.1
        if prof is None and step_s:
            r += step_s * 0.5
        return r

    t_c = t_d = 0.0
    ok_all = True
    K = 0
    lens = None
    while K < args.steps:
        left = args.budget_s - (time.perf_counter() - t_start) - reserve()
        if K > 0 and step_s and left < step_s * 1.05:
            break
        # a part run profiles its one timed step instead of a second pass
        tc, td, lens, ok, p_step = step(profile=part is not None and prof is None)
        if p_step is not None:
            prof = p_step
        K += 1
        step_s = tc + (0 if args.no_decompress else td)
        log(f"timed step {K}: compress {tc:.3f} s, decompress {td:.3f} s, round trip {ok}")
        t_c += tc
        t_d += td
        ok_all = ok_all and (ok is not False)
    if K < args.steps:
        log(f"timed {K} of {args.steps} requested steps (wall budget {args.budget_s:.0f} s)")
    comp_mb_s = n * K / t_c / 1e6
    dec_mb_s = n * K / t_d / 1e6 if not args.no_decompress else None
    ratio = n / container_bytes(lens, n_chunks)

    if prof is None:  # no warmup step: profile one compress pass now
        log("compress pass with kernel profiling")
        codec.profile(True)
        codec.profile_reset()
        codec.compress_device(d_data, n, chunk, d_pay, cap)
        torch.cuda.synchronize()
        prof = codec.profile_read()
        codec.profile(False)

    # per-class kernel times of the compress (HIP events on the launch stream)
    kernel_ms = {k: round(v["ms"], 3) for k, v in prof.items() if v["launches"]}
    g = prof["gemm"]
    peak_mm = PEAK_TFLOPS[prec]
    gemm_launch_us = g["ms"] * 1e3 / max(g["launches"], 1)
    sc = prof["scan"]
    r_dt = -(-d // 16)
    rb = 8 if r_dt <= 8 else (16 if r_dt <= 16 else 32)
    ta = "float" if prec == "fp32" else "unsigned short"
    comp_lanes = min(args.warm_start, n_chunks) if args.warm_start else n_chunks
    if comp_lanes * 2 * d < 64 * 1024:  # under one wave per SIMD: the token-blocked form
        scan_kernel = f"boa::scan_chunk_tblk_kernel<{ds}, {rb}, {ta}>"
    else:
        scan_kernel = f"boa::scan_chunk_sload_kernel<{ds}, {rb}, {str(r_dt == rb).lower()}, {ta}>"

    # The decode step's kernels on directly launched steps (boa_step_batch)
    # after the timed region, each launch timed by the HIP events its
    # dispatch packet carries (hipExtLaunchKernelGGL: the kernel's own span,
    # as rocprofv3 measures it).
    dec = None
    dec_cls = {}
    if not args.no_decompress:
        log("decode-step kernel profile (32 directly launched steps)")
        lanes = n_chunks
        prof_dec = decode_step_profile(codec, lanes)
        plan = codec.decode_plan(lanes)
        dec = {"lanes": lanes, "steps": 32, "launch": "direct, HIP events in each dispatch",
               "plan": plan,
               "kernel_us_per_step": {k: round(v["us_per_step"], 2) for k, v in prof_dec.items()}}
        # A persistent decode (d_model 64) runs the whole batch in one
        # kernel, not these step kernels: its candidate below is the whole
        # decompress.
        if not plan["persistent"]:
            for k, v in prof_dec.items():
                n_l = v["launches_per_step"]
                dec_cls[k] = dict(avg_us=v["us_per_step"] / n_l, launches_per_step=n_l,
                                  work_per_launch=v["work_per_step"] / n_l)
            log("decode coder-step profile (64 profiled decompress steps)")
            dc = decode_coder_profile(codec, torch, data, chunk, n_chunks)
            # the unfused coder step reads each lane's 1 KB logits row; with
            # head.2 fused in (from 2048 lanes) its work is counted in FLOP
            if dc["launches"] and not plan["fused_head"]:
                dec_cls["decode"] = dict(avg_us=dc["ms"] * 1e3 / dc["launches"], launches_per_step=1,
                                         work_per_launch=dc["work"] / dc["launches"])
                dec["kernel_us_per_step"]["decode"] = round(dec_cls["decode"]["avg_us"], 2)

    # Rooflines of the kernels that take most of a round trip; `roofline`
    # is the one with the largest total time per step (compress: its
    # launches in the profiled pass; decode: launches per step x the launch
    # time x the chunk - 1 steps of the cold single-batch decode).  Every
    # launch time comes from the HIP events in its dispatch packet.
    steps_per_dec = chunk - 1
    cands = {}

    def add(name, kernel, bound, work_per_launch, avg_us, launches_per_rt, unit_peak, **extra):
        if avg_us <= 0 or launches_per_rt <= 0:
            return
        if bound == "mfma":
            ach = work_per_launch / (avg_us * 1e-6) / 1e12
            e = roofline_entry(kernel, "mfma", ach, unit_peak, "TFLOP/s", avg_us, work_per_launch,
                               "flop_per_launch", **extra)
        else:
            ach = work_per_launch / (avg_us * 1e-6) / 1e9
            e = roofline_entry(kernel, "hbm", ach, PEAK_HBM_GBS, "GB/s", avg_us, work_per_launch,
                               "bytes_per_launch", **extra)
        e["s_per_round_trip"] = round(avg_us * 1e-6 * launches_per_rt, 3)
        e["launches_per_round_trip"] = round(launches_per_rt)
        cands[name] = e

    add("compress GEMM", GEMM_KERNEL[prec], "mfma", g["work"] / max(g["launches"], 1),
        gemm_launch_us, g["launches"], peak_mm,
        traffic=gemm_traffic_bytes() if workload == "c2" else None)
    scan_us = sc["ms"] * 1e3 / max(sc["launches"], 1)
    scan_extra = {}
    vpe = SCAN_VALU_PER_ELEMENT.get((prec, ds), 0)
    if vpe and sc["launches"] and "sload" in scan_kernel:
        # the scan's other bound: VALU issue.  Elements per launch from the
        # algorithmic bytes (4 (3 di + R) per row in fp32, 2 (3 di) + 2 R in bf16)
        rows = sc["work"] / sc["launches"] / ((4 if prec == "fp32" else 2) * (3 * 2 * d + r_dt + 2 * ds))
        wi = rows * 2 * d * vpe / 64 / (scan_us * 1e-6)
        scan_extra["valu"] = {"bound": "valu issue", "instr_per_element": vpe,
                              "achieved_g_wave_instr_s": round(wi / 1e9, 1),
                              "peak_g_wave_instr_s": round(VALU_ISSUE_PEAK / 1e9, 1),
                              "frac": round(wi / VALU_ISSUE_PEAK, 3),
                              "note": "instr_per_element counted from the compiled loop; peak "
                                      "= the published fp32 vector peak (157.3 TFLOP/s) in wave64 "
                                      "FMA instructions"}
    add("compress scan", scan_kernel, "hbm", sc["work"] / max(sc["launches"], 1), scan_us,
        sc["launches"], None, **scan_extra)
    hc = prof["head_cdf"]
    if hc["launches"]:
        hk = ("boa::gemm_f32_kernel<64, 256, 4, 4, 16, 3>" if prec == "fp32" else
              "boa::gemm_bf16_kernel<256, 256, 4, 4, 64, 1|2, 3>")
        add("compress head.2 + CDF", hk + " (head.2 with the CDF epilogue)", "mfma",
            hc["work"] / hc["launches"], hc["ms"] * 1e3 / hc["launches"], hc["launches"], peak_mm)
    co = prof["coder"]
    if co["launches"]:
        # range encoder (8 B of (low, prob) per symbol read, compressed words
        # written) and the payload compaction (words read and written)
        add("compress coder", "boa::rc_encode_tile_kernel + boa::compact_kernel", "hbm",
            co["work"] / co["launches"], co["ms"] * 1e3 / co["launches"], co["launches"], None)
    kn = {"dec_lngemm": ("decode LayerNorm GEMMs", "boa::dec_ln_gemm_kernel<1|2, d/16, *> "
                         "(LN1 + in_proj + conv, LN2 + FF1 + GELU)", "mfma"),
          "dec_gemm": ("decode GEMMs", "boa::dec_gemm_kernel / dec_b16_gemm* (x_proj, out_proj, "
                       "FF2, heads)", "mfma"),
          "dec_scan": ("decode scan", "boa::dec_xscan_kernel / dec_scan_kernel / dec_b16_scan_kernel",
                       "hbm"),
          "decode": ("decode coder step", "boa::decode_step_kernel (CDF, search, coder advance) / "
                     "dec_head_step_kernel (head.2 fused in)", "hbm")}
    c2_lanes = args.config == "c2" and not args.warm_start and n_chunks == 1000
    for k, (name, kernel, bound) in kn.items():
        if k in dec_cls:
            v = dec_cls[k]
            extra = {"traffic": dec_ln_gemm_traffic_bytes()} if k == "dec_lngemm" and c2_lanes else {}
            add(name, kernel, bound, v["work_per_launch"], v["avg_us"],
                v["launches_per_step"] * steps_per_dec, peak_mm, **extra)
    if dec is not None and dec["plan"]["persistent"] and K:
        # model FLOPs per token: in_proj, x_proj, dt_proj, out_proj, FF1, FF2
        # per layer, then head.1 and head.2
        di, r_dt = 2 * d, -(-d // 16)
        macs = L * (d * 2 * di + di * (r_dt + 2 * ds) + r_dt * di + di * d + 8 * d * d) + d * d + d * 256
        flops = 2.0 * macs * (n - n_chunks)  # one model step per byte after a chunk's first
        add("decode (persistent kernel)", "boa::dec_persist_kernel (every step of the batch in "
            "one launch)", "mfma", flops, t_d / K * 1e6, 1, peak_mm)
    dom = max(cands, key=lambda k: cands[k]["s_per_round_trip"])
    roofline = dict(cands[dom])
    roofline["class"] = dom

    host = None
    if not args.no_host_path:
        left = args.budget_s - (time.perf_counter() - t_start) - (0 if args.no_cpu else 45.0)
        if step_s and left > step_s * 1.1:
            log("host-buffer round trip (PCIe-inclusive)")
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            blob = codec.compress(data, chunk_size=chunk)
            t1 = time.perf_counter()
            back = codec.decompress(blob) if not args.no_decompress else data
            t2 = time.perf_counter()
            host = {"compress_mb_s": round(n / (t1 - t0) / 1e6, 4),
                    "decompress_mb_s": round(n / (t2 - t1) / 1e6, 4) if not args.no_decompress else None,
                    "container_bytes": len(blob), "roundtrip_ok": back == data,
                    "container_matches_device_path": len(blob) == container_bytes(lens, n_chunks),
                    "span": "input bytes in host memory -> BOA2 container in host memory "
                            "(H2D, D2H and the container write included)"}
            ok_all = ok_all and host["roundtrip_ok"]
        else:
            log("host-buffer round trip skipped (wall budget)")

    cpu = None
    if not args.no_cpu:
        info = cpu_info()
        threads = args.cpu_threads or int(info["omp_num_threads"] or 0) or info["affinity"]
        sample_chunks = min(args.cpu_sample_chunks, n_chunks)
        log(f"cpu baseline: {sample_chunks} chunks x {args.cpu_sample_len} B on {threads} threads")
        cb = cpu_baseline(weights, data, chunk, n_chunks, sample_chunks, args.cpu_sample_len,
                          threads, d, L, ds, bf16=prec == "bf16")
        cpu = {"value": round(cb["compress_mb_s"], 5), "unit": "MB/s", "cores": threads,
               "kind": "port",
               "sample": f"first {args.cpu_sample_len} B of each of the first {sample_chunks} chunks "
                         f"({cb['bytes']} B), oracle/refcpu compress (OpenMP over chunks)",
               "decompress_value": round(cb["decompress_mb_s"], 5),
               "compress_s": round(cb["compress_s"], 2), "decompress_s": round(cb["decompress_s"], 2),
               "isa": {"v4": "x86-64-v4 (AVX-512)", "v3": "x86-64-v3 (AVX2 + FMA)"}.get(cb["isa"], cb["isa"]),
               "build": f"gcc -O3 -march=x86-64-{cb['isa']} -ffp-contract=off -fopenmp ({cb['lib']})",
               "host": info,
               "threads_rule": "OMP_NUM_THREADS of the GPU box (its CPU share for one GPU), "
                               "else every core in the process's affinity mask"}

    out = {
        "metric": METRIC,
        "value": round(comp_mb_s, 4),
        "unit": "MB/s",
        "n_gpus": 1,
        "steps": K,
        "steps_requested": args.steps,
        "warmup": warm_done,
        "warmup_requested": args.warmup,
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
                   "input": f"synth.gen_{args.config}",
                   **({"part": part} if part else {})},
        "compress_mb_s": round(comp_mb_s, 4),
        "decompress_mb_s": round(dec_mb_s, 4) if dec_mb_s else None,
        "value_span": "device-resident: input in HBM -> compacted payload in HBM (and back)",
        "compression_ratio": round(ratio, 5),
        "roundtrip_ok": ok_all,
        "compress_kernel_ms": kernel_ms,
        "roofline": roofline,
        "rooflines": cands,
        "decode_step": dec,
        "host_path": host,
        "cpu_baseline": cpu,
        "wall_s": round(time.perf_counter() - t_start, 1),
    }
    if cpu:
        out["speedup_vs_cpu_compress"] = round(comp_mb_s / cpu["value"], 1)
    print(json.dumps(out), flush=True)
    codec.set_progress(None)
    codec.close()
    return 0 if ok_all else 1


if __name__ == "__main__":
    sys.exit(main())
