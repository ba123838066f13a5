#!/usr/bin/env python3
"""Encoder RTFx of the Parakeet-TDT-0.6B-v3-shaped FastConformer on one MI355X.

A step is one encoder call over 60 s of synthetic audio: the 128-bin log-mel (6001 frames, resident in
HBM before the timed region) → 8× subsampling → 24 Conformer blocks (d 1024, 8 heads of 128, relative
positions, FFN 4096, conv kernel 9) → the joint's encoder projection, all GEMM weights q8_0 (random
N(0, 0.02), written as a GGUF file and loaded through the C ABI).  value = audio seconds per second
of encoder time (RTFx), timed over --steps calls after --warmup.

`roofline` is the dominant kernel of the step (by total time in a profiled step: HIP events around each
launch on the library's stream), its algorithmic flops (2·M·N·K summed over its launches) over its
measured time, against MI355X's dense fp16 MFMA peak.  `cpu_baseline` is the C parity oracle (the
restated wavo CPU backend, portable f16-rounded arithmetic, AVX2+FMA, OpenMP) on the same model and
mel, one full call, timed on this host.
"""

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encoder RTFx (audio s/s) at 1 MI355X; q8_0 GEMM % MFMA peak; GEMV % HBM BW"
PEAK_F16 = 2500.0     # TFLOP/s, MI355X dense fp16 MFMA
PEAK_HBM = 8000.0     # GB/s


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seconds", type=float, default=60.0, help="audio per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X: this build has no multi-GPU path (asked for {max(args.gpus, world)}). "
              "Segments of long audio shard across GPUs with no exchange step; run one process per GPU.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np

    import wavo_amd as wa
    from wavo_amd import synth

    t0 = time.time()
    path = synth.model_path("parakeet")
    log(f"model {path} ready in {time.time() - t0:.1f} s")
    gpu = wa.Gpu(0)
    t0 = time.time()
    model = wa.Model(gpu, path)
    log(f"loaded on {gpu.name} ({gpu.cus} CUs) in {time.time() - t0:.1f} s")
    pcm = synth.audio(args.seconds, seed=1)
    mel = synth.parakeet_mel(pcm)
    mel_frames = mel.shape[0]
    frames, width = model.frames(mel_frames)
    melb = gpu.upload(mel)
    outb = gpu.buffer(frames * width)

    for _ in range(args.warmup):
        model.encode_device(melb, mel_frames, outb)
    gpu.sync()
    log(f"warmup done ({args.warmup} steps), timing {args.steps}")
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.encode_device(melb, mel_frames, outb)
    gpu.sync()
    dt = (time.perf_counter() - t0) / args.steps
    rtfx = args.seconds / dt
    log(f"{dt * 1e3:.3f} ms per step, RTFx {rtfx:.0f}")

    # One profiled step: per-kernel time and algorithmic work.
    gpu.profile(True)
    model.encode_device(melb, mel_frames, outb)
    prof = gpu.profile_read()
    gpu.profile(False)
    total_ms = sum(k["ms"] for k in prof)
    by_family = {}
    for k in prof:
        fam = k["kernel"].split("_")[0] if k["kernel"].startswith("gemm") else k["kernel"]
        by_family[fam] = by_family.get(fam, 0.0) + k["ms"]
    dom = max(prof, key=lambda k: k["ms"])
    q8 = [k for k in prof if k["kernel"].startswith("gemm_q8_0")]
    gemm_flops = sum(k["flops"] for k in q8)
    gemm_ms = sum(k["ms"] for k in q8)
    achieved = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
    roofline = {
        "bound": "mfma",
        "kernel": dom["kernel"],
        "achieved": round(achieved, 2),
        "peak": PEAK_F16,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_F16, 4),
        "traffic": None,
        "launches_per_step": dom["launches"],
        "avg_launch_us": round(dom["ms"] * 1e3 / dom["launches"], 2),
        "flops_per_launch": dom["flops"] / dom["launches"],
        "all_q8_0_gemm": {"ms": round(gemm_ms, 4), "tflops": round(gemm_flops / (gemm_ms * 1e-3) / 1e12, 2),
                          "frac": round(gemm_flops / (gemm_ms * 1e-3) / 1e12 / PEAK_F16, 4)},
    }
    # The step's kernels, summed per family (ms per step), and what the launches leave out.
    breakdown = {k: round(v, 4) for k, v in sorted(by_family.items(), key=lambda x: -x[1])}
    breakdown["gaps"] = round(dt * 1e3 - total_ms, 4)

    cpu = None
    if not args.no_cpu:
        import oracle

        om = oracle.Model(path)
        log(f"CPU baseline: oracle on {oracle.lib().ox_threads()} threads")
        t0 = time.perf_counter()
        want = om.encode(mel)
        cdt = time.perf_counter() - t0
        got = gpu.read(outb, (frames, width))
        err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
        cpu = {"value": round(args.seconds / cdt, 3), "unit": "audio s/s", "cores": oracle.lib().ox_threads(),
               "kind": "port", "seconds": round(cdt, 3),
               "sample": f"one full encoder call on the same {args.seconds:.0f} s mel and model (restated wavo CPU "
                         f"backend, portable f16-rounded GEMM, AVX2+FMA, OpenMP); GPU-vs-CPU rel L2 {err:.2e}"}
        log(f"CPU {cdt:.2f} s, rel L2 {err:.2e}")

    out = {
        "metric": METRIC,
        "value": round(rtfx, 2),
        "unit": "audio s/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded audio → log-mel; random-init N(0,0.02) weights, q8_0 GGUF)",
        "config": {"workload": "parakeet-tdt-0.6b-v3-shaped encoder, 60 s audio, q8_0 (BASELINE configs[1])",
                   "audio_s": args.seconds, "mel_frames": mel_frames, "encoder_frames": frames,
                   "layers": model.layers, "d_model": model.d, "weights": "q8_0"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "breakdown_ms": breakdown,
    }
    print(json.dumps(out), flush=True)
    gpu.close()


if __name__ == "__main__":
    main()
