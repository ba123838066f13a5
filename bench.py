#!/usr/bin/env python3
"""Encoder RTFx of the Parakeet-TDT-0.6B-v3-shaped FastConformer on one MI355X.

A step is one encoder call over 60 s of synthetic audio: the 128-bin log-mel (6001 frames, resident in
HBM before the timed region) → 8× subsampling → 24 Conformer blocks (d 1024, 8 heads of 128, relative
positions, FFN 4096, conv kernel 9) → the joint's encoder projection, all GEMM weights q8_0 (random
N(0, 0.02), written as a GGUF file and loaded through the C ABI).  value = audio seconds per second
of encoder time (RTFx), timed over --steps calls after --warmup (HIP events on the library's stream
around the whole timed region; the calls after the second replay a recorded HIP graph of the step).

`roofline` is the dominant q8_0 GEMM of the step: the (kernel variant, call shape) with the most time
in a profiled step.  Its average launch duration is measured by launching that exact configuration
(same tile plan, m × n × k, epilogue and output type; random q8_0 weights of the same shape) 50 times
back to back between two HIP events on the library's stream — events around every single launch would
add their own few microseconds to each — and `achieved` = 2·m·n·k per launch over that duration, against
MI355X's dense fp16 MFMA peak.  A k-split configuration is timed as its GEMM kernel alone, as in the step
(where the next kernel, fused with the LayerNorm, adds the partial sums).  `traffic` is that launch's HBM bytes from rocprofv3 FETCH_SIZE /
WRITE_SIZE passes (profiles/), when a summary for the same configuration is committed there.

`gemv` is the Whisper-large-v3-turbo decoder's per-token matrix-vector products (q8_0; 4 layers of
qkv 3840×1280, self_out / cross_q / cross_out 1280×1280, fc1 5120×1280, fc2 1280×5120, and the
51866-row head), timed cold: two copies of the weights (2 × 168 MB, past the 256 MB Infinity Cache)
alternate, and achieved bytes per second of the weights as stored is reported against HBM peak;
`gemv.head` is the head alone, and `gemv.decode_step` the whole decoder step (embedding, 4 layers of
norms, GEMVs, self- and cross-attention, the head) replayed as one recorded pass per token for 224
tokens, with the weights left in the Infinity Cache between tokens as a decode loop leaves them.

`cpu_baseline` is the C parity oracle (the restated wavo CPU backend, portable f16-rounded arithmetic,
AVX2+FMA, OpenMP) on the same model and mel, one full call, timed on this host.
"""

import argparse
import json
import os
import re
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "encoder RTFx (audio s/s) at 1 MI355X; q8_0 GEMM % MFMA peak; GEMV % HBM BW"
PEAK_F16 = 2500.0     # TFLOP/s, MI355X dense fp16 MFMA
PEAK_HBM = 8000.0     # GB/s
GEMM_NAME = re.compile(r"^gemm_(\w+?)_(\d+)x(\d+)_w(\d+)x(\d+)_n(\d+)(_s\d)? (\d+)x(\d+)x(\d+) e(\d+) (f16|f32) w(\d+)$")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_region(gpu, fn, reps):
    """Milliseconds per call of fn() over `reps` back-to-back calls between two events."""
    gpu.profile(2)
    gpu.region_begin("batch")
    for _ in range(reps):
        fn()
    gpu.region_end()
    ms = gpu.profile_read()[0]["ms"]
    gpu.profile(0)
    return ms / reps


def gemm_replay(gpu, name, reps=50):
    """Re-launches the GEMM configuration `name` (a profile record) back to back; returns us/launch."""
    import numpy as np

    import wavo_amd as wa
    from wavo_amd import gguf

    g = GEMM_NAME.match(name)
    tn, bm, bn, wm, wn, ns, split, m, n, k, epi, out, width = g.groups()
    wtype = {"q8_0": wa.Q8_0, "q4_0": wa.Q4_0, "f16": wa.F16}[tn]
    rng = np.random.default_rng(5)
    w = gguf.encode(rng.standard_normal(int(n) * int(k), dtype=np.float32) * np.float32(0.02), wtype)
    f16 = out == "f16"
    plan = f"{bm},{bn},{wm},{wn},{ns},{split[2:] if split else 1}"
    import wavo_amd

    g2 = wavo_amd.Gpu(0)
    g2.tune("gemm_plan", plan)  # the same launch plan as in the step
    # A split GEMM's kernel alone, as it runs in the step (where the following fused LayerNorm kernel
    # adds the partial sums); a C-ABI call would add its own finishing kernel.
    g2.tune("gemm_kernel_only", 1)
    lin2 = g2.linear([(w, wtype, int(k), int(n))], np.zeros(int(width), np.float32))
    a2 = g2.upload(rng.standard_normal((int(m), int(k)), dtype=np.float32).astype(np.float16))
    c2 = g2.buffer(int(m) * int(width))
    run = lambda: g2.gemm_h(a2, lin2, c2, int(m), int(epi), 0.5, out16=f16)
    for _ in range(5):
        run()
    g2.sync()
    us = time_region(g2, run, reps) * 1e3
    del lin2, a2, c2
    g2.close()
    return us, 2.0 * int(m) * int(n) * int(k)


def gemv_cold(gpu):
    """Whisper decoder GEMVs per token, q8_0, two weight copies alternating (cold)."""
    import numpy as np

    import wavo_amd as wa
    from wavo_amd import gguf

    d, ff, vocab, layers = 1280, 5120, 51866, 4
    shapes = []
    for _ in range(layers):
        shapes += [(3 * d, d, wa.BIAS), (d, d, wa.RESIDUAL), (d, d, wa.BIAS), (d, d, wa.RESIDUAL),
                   (ff, d, wa.GELU), (d, ff, wa.RESIDUAL)]
    shapes.append((vocab, d, wa.BIAS))
    rng = np.random.default_rng(9)
    raw = {}
    for (n, k, _) in set(shapes):
        raw[(n, k)] = gguf.encode(rng.standard_normal(n * k, dtype=np.float32) * np.float32(0.02), wa.Q8_0)
    copies = [[gpu.linear([(raw[(n, k)], wa.Q8_0, k, n)], np.zeros(n, np.float32)) for (n, k, _) in shapes]
              for _ in range(2)]
    x = gpu.upload(rng.standard_normal(ff, dtype=np.float32))
    y = gpu.upload(np.zeros(vocab + 64, np.float32))
    wbytes = sum(n * k // 32 * 34 for (n, k, _) in shapes)

    def token(i):
        for lin, (n, k, e) in zip(copies[i % 2], shapes):
            gpu.gemv(x, lin, y, e, 1.0)

    for i in range(4):
        token(i)
    gpu.sync()
    # A token's GEMVs as one recorded pass per weight copy (Gpu::record), as a decoder step submits
    # them: the time is the GPU's, not the launches' from Python.
    passes = []
    for i in range(2):
        gpu.record_begin()
        token(i)
        passes.append(gpu.record_end())
    for p in passes:
        p.replay()
    reps = 20
    state = {"i": 0}

    def one():
        passes[state["i"] % 2].replay()
        state["i"] += 1

    ms = time_region(gpu, one, reps)
    for p in passes:
        p.free()
    # The head alone (70.6 MB), cold: one launch per call (a one-node recorded pass costs more to
    # launch than the kernel runs).
    head = [c[-1] for c in copies]
    st2 = {"i": 0}

    def one_head():
        gpu.gemv(x, head[st2["i"] % 2], y, wa.BIAS)
        st2["i"] += 1

    for _ in range(4):
        one_head()
    hms = time_region(gpu, one_head, 40)
    hbytes = vocab * d // 32 * 34
    out = {"workload": "whisper-large-v3-turbo decoder GEMVs per token, q8_0, cold (2 weight copies of 168 MB alternate), "
                       "each token's 25 GEMVs replayed as one recorded pass",
           "launches_per_token": len(shapes), "us_per_token": round(ms * 1e3, 2), "weight_bytes": wbytes,
           "achieved": round(wbytes / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM, "unit": "GB/s",
           "frac": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_HBM, 4),
           "head": {"shape": f"{vocab}x{d}", "us": round(hms * 1e3, 2), "bytes": hbytes,
                    "achieved": round(hbytes / (hms * 1e-3) / 1e9, 1),
                    "frac": round(hbytes / (hms * 1e-3) / 1e9 / PEAK_HBM, 4)}}
    del copies
    return out


def decode_steps(gpu, tokens=224):
    """Whisper-large-v3-turbo-shaped decoder steps (4 layers, d 1280, 20 heads, 51866-token head, cross
    attention over 1500 encoder frames, q8_0), `tokens` steps back to back after one warm-up pass."""
    import numpy as np

    import wavo_amd as wa
    from wavo_amd import synth

    t0 = time.time()
    path = synth.model_path("whisper")
    m = wa.Model(gpu, path)
    log(f"whisper model ready in {time.time() - t0:.1f} s")
    cfg = synth.CONFIGS["whisper"]
    frames, d, vocab = cfg["frames"], cfg["d"], cfg["vocab"]
    enc = np.random.default_rng(3).normal(0, 1, (frames, d)).astype(np.float32)
    eb = gpu.upload(enc)
    lb = gpu.buffer(vocab if vocab % 32 == 0 else (vocab + 63) // 64 * 64)
    m.whisper_begin(eb, frames)
    ids = np.random.default_rng(4).integers(0, vocab, tokens)
    for pos in range(8):  # the first two calls record the step; later ones replay it
        m.whisper_step(int(ids[pos]), pos, lb)
    gpu.sync()
    m.whisper_begin(eb, frames)
    state = {"pos": 0}

    def one():
        m.whisper_step(int(ids[state["pos"]]), state["pos"], lb)
        state["pos"] += 1

    ms = time_region(gpu, one, tokens)
    m.free()
    return {"workload": f"whisper-large-v3-turbo-shaped decoder step (4 layers, d {d}, {cfg['dec_heads']} heads, "
                        f"{vocab}-token head, cross attention over {frames} frames, q8_0), {tokens} steps back to back "
                        "(weights stay in the MALL between tokens), one recorded pass per step",
            "us_per_token": round(ms * 1e3, 2), "tokens_per_s": round(1e3 / ms, 1)}


def traffic_for(name):
    """HBM bytes per launch for this GEMM configuration from a committed rocprofv3 summary, if any."""
    path = os.path.join(ROOT, "profiles", "gemm_traffic.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic ") and name in line:
            try:
                return json.loads(line.split(" ", 1)[1].split(" | ", 1)[1])
            except (ValueError, IndexError):
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--seconds", type=float, default=60.0, help="audio per step")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-gemv", action="store_true", help="skip the decoder GEMV and decoder step measurements")
    ap.add_argument("--replay", metavar="NAME", default=None,
                    help="only the back-to-back launches of this GEMM configuration (a roofline.kernel value), "
                         "for rocprofv3 passes over exactly those launches")
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

    if args.replay:
        if not GEMM_NAME.match(args.replay):
            sys.exit(f"--replay takes a GEMM configuration name like the bench line's roofline.kernel: {args.replay!r}")
        us, flops = gemm_replay(None, args.replay)
        print(json.dumps({"replayed": args.replay, "us_per_launch": round(us, 3),
                          "tflops": round(flops / (us * 1e-6) / 1e12, 2)}), flush=True)
        return

    t0 = time.time()
    path = synth.model_path("parakeet")
    log(f"model {path} ready in {time.time() - t0:.1f} s")
    gpu = wa.Gpu(0)
    t0 = time.time()
    model = wa.Model(gpu, path)
    log(f"loaded on {gpu.name or 'gfx950'} ({gpu.cus} CUs) in {time.time() - t0:.1f} s")
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
    ms_ev = time_region(gpu, lambda: model.encode_device(melb, mel_frames, outb), args.steps)
    wall = (time.perf_counter() - t0) / args.steps
    dt = ms_ev * 1e-3
    rtfx = args.seconds / dt
    log(f"{dt * 1e3:.3f} ms per step (events; wall {wall * 1e3:.3f}), RTFx {rtfx:.0f}")

    # One profiled step: per-kernel launches and algorithmic work (events around each launch).
    gpu.profile(1)
    model.encode_device(melb, mel_frames, outb)
    prof = gpu.profile_read()
    gpu.profile(0)
    gemms = [k for k in prof if GEMM_NAME.match(k["kernel"])]
    dom = max(gemms, key=lambda k: k["ms"])
    us, flops = gemm_replay(gpu, dom["kernel"])
    log(f"dominant GEMM {dom['kernel']}: {dom['launches']} launches per step, {us:.2f} us per launch back to back")

    achieved = flops / (us * 1e-6) / 1e12
    fam = {}
    for k in prof:
        f = k["kernel"].split(" ")[0]
        e = fam.setdefault(f, [0, 0.0])
        e[0] += k["launches"]
        e[1] += k["ms"]
    q8 = [k for k in gemms if k["kernel"].startswith("gemm_q8_0")]
    q8_flops = sum(k["flops"] for k in q8)
    q8_ms = sum(k["ms"] for k in q8)
    roofline = {
        "bound": "mfma",
        "kernel": dom["kernel"],
        "achieved": round(achieved, 2),
        "peak": PEAK_F16,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_F16, 4),
        "traffic": traffic_for(dom["kernel"]),
        "launches_per_step": dom["launches"],
        "avg_launch_us": round(us, 2),
        "flops_per_launch": flops,
        "timing": "50 back-to-back launches of this configuration between two HIP events on the library's stream",
        "all_q8_0_gemm_profiled": {"launches": sum(k["launches"] for k in q8), "ms": round(q8_ms, 4),
                                   "tflops_incl_event_overhead": round(q8_flops / (q8_ms * 1e-3) / 1e12, 2)},
    }
    breakdown = {f: {"launches": n, "ms": round(ms, 4)} for f, (n, ms) in sorted(fam.items(), key=lambda x: -x[1][1])}

    gemv = None if args.no_gemv else gemv_cold(gpu)
    if gemv:
        log(f"GEMV per token {gemv['us_per_token']} us, {gemv['achieved']} GB/s ({gemv['frac'] * 100:.1f}% of HBM)")
        gemv["decode_step"] = decode_steps(gpu)
        log(f"decoder step {gemv['decode_step']['us_per_token']} us per token")

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
        "gemv": gemv,
        "cpu_baseline": cpu,
        "profiled_step_ms": breakdown,
    }
    print(json.dumps(out), flush=True)
    model.free()
    gpu.close()


if __name__ == "__main__":
    main()
