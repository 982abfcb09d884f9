#!/usr/bin/env python3
"""Benchmark of the MI355X Voxtral frame loop (one JSON line on stdout).

Workload (the headline configuration): the full 26-layer backbone
(dim 3072, 32/8 heads of 128, FFN 9216, random-init f16 weights N(0,0.02)),
batch 1, decoding at context 512 after a real prefill of a seeded random
512-token prefix (ids uniform over 131072).  A step is one complete decode
step (26 layers + final norm; the LM head is off, as in generate()), with
all inputs resident in HBM.  value = decode steps (frames) per second.

Also reported: the full frame loop (backbone step + 3-layer flow-matching
CFG Euler loop, greedy semantic code on the device, 500 frames from
context 512) as x-real-time (one frame = 80 ms of audio), generate() end to
end (prompt, frames, codec decode) per sampling mode, the codec decoder on
its own, the roofline of the dominant kernel, and the CPU oracle timed on
the host cores.
Diagnostics go to stderr.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "webgpu-voxtral_amd"))

METRIC = "backbone decode frames/s @ctx512 + % HBM roofline, full frame loop x-realtime"
HBM_PEAK_GBPS = 8000.0
CTX = 512
LAYERS = 26
# algorithmic HBM bytes (f16 weights; f32 KV cache, the reference's precision)
LAYER_WEIGHT_BYTES = 232_796_160          # q,k,v,o,w1,w2,w3 + 2 norms
FM_EULER_BYTES = 698_836_992              # 3 FM layers + input/acoustic proj + norm
FM_FRAME_BYTES = 69_992_448               # semantic head + llm projection
EMB_CODES_BYTES = 37 * 3072 * 2           # 37-row multi-codebook sum


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def codec_flops(T):
    """Algorithmic flops of the codec decoder for T frames (1 multiply-add =
    2 flops): input conv 292*3 -> 1024; per stage 2 layers of q,k,v,o
    (1024^2 each), gate/up (2 x 4096x1024), down (1024x4096) over the
    stage's tokens plus the windowed attention; stride-2 transposed convs
    (2 taps x 1024 channels per output); output conv 1024*7 -> 240."""
    f = 2 * T * 1024 * 292 * 3
    tt = T
    for s, w in enumerate((2, 4, 8, 16)):
        f += 2 * 2 * tt * (4 * 1024 * 1024 + 3 * 4096 * 1024)
        f += 2 * 2 * tt * 8 * 128 * w * 2
        if s < 3:
            f += 2 * (2 * tt) * 1024 * 2048
            tt *= 2
    f += 2 * tt * 240 * 1024 * 7
    return f


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (counters scaled by a device copy of known size), or None."""
    path = os.path.join(ROOT, "profiles", "backbone_gemv_ctx512_pmc_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if parts[:2] == ["traffic_bytes_per_launch", kernel]:
                    return int(parts[2])
    except OSError:
        pass
    return None


def trace_avg_us(kernel):
    """Average duration per dispatch of `kernel` in the committed rocprofv3
    --kernel-trace --stats summary of the decode step, or None."""
    path = os.path.join(ROOT, "profiles", "backbone_decode_ctx512_kernel_trace.md")
    try:
        with open(path) as f:
            for line in f:
                parts = line.split()
                if parts[:2] == ["trace_avg_us", kernel]:
                    return float(parts[2])
    except OSError:
        pass
    return None


def kv_bytes_per_key(kv_elem):
    return LAYERS * 2 * 1024 * kv_elem    # K and V rows of every layer


def step_bytes(keys, kv_elem=4):
    """weights + K/V rows read for `keys` keys + the new K/V row written"""
    return LAYERS * LAYER_WEIGHT_BYTES + kv_bytes_per_key(kv_elem) * (keys + 1)


def prefilled_engine(V, kv_f16):
    eng = V.VoxtralEngine(V.default_config(kv_f16=int(kv_f16)), max_seq_len=4096).init()
    eng.init_synthetic(0, 0.02)
    toks = np.random.default_rng(0).integers(0, 131072, CTX)
    eng.prefill(toks)
    assert eng.position == CTX
    return eng


# flops of one token through the 26 layers' projections (2 per weight)
TOKEN_FLOP = 2 * LAYERS * (6144 * 3072 + 3072 * 4096 + 2 * 9216 * 3072 + 3072 * 9216)
MFMA_PEAK_F16 = 2.5e15  # dense f16 MFMA, MI355X


def measure_prompt(eng, reps=5, decode=True):
    """The 256-token prompt with 64 voice rows N(0,1) spliced at offset 2,
    prefilled as batched GEMMs, then (decode) 500 decode steps over the
    growing context (257..756 keys)."""
    toks = np.random.default_rng(1).integers(0, 131072, 256)
    voice = np.random.default_rng(2).standard_normal((64, 3072)).astype(np.float32)
    times = []
    for _ in range(reps):
        eng.reset()
        t = time.perf_counter()
        eng.prefill(toks, 2, 64, voice)
        times.append(time.perf_counter() - t)
    pf = float(np.median(times[1:]))
    useful = TOKEN_FLOP * 256
    issued = useful * 2  # hi and lo halves of the activations
    out = {"prefill_ms": round(pf * 1e3, 3), "prefill_tokens_per_s": round(256 / pf, 1),
           "useful_TFLOPs": round(useful / pf / 1e12, 2),
           "mfma_issued_TFLOPs": round(issued / pf / 1e12, 2),
           "mfma_frac_of_peak": round(issued / pf / MFMA_PEAK_F16, 4)}
    if not decode:
        return out
    # each step's input is the previous step's W.normed (the precomputed-
    # embedding path), the prompt configuration's decode tail
    ms = eng.time_backbone_steps(500, feedback=True)
    fps = 500 * 1000.0 / ms
    return {**out,
            "decode_steps": 500, "decode_ms_per_step": round(ms / 500, 5),
            "decode_frames_per_s": round(fps, 2),
            "note": "prefill timed on the host clock around vx_prefill (host copies of 256 ids and "
                    "64 voice rows included), median of 4 after 1 warm-up; decode steps fed "
                    "back through W.normed as the precomputed embedding, HIP events"}


def measure_codec(eng, T=250, reps=10, warm=3):
    """codecDecode of T frames of random codes, wall time per call (median
    of reps after warm calls)."""
    rng = np.random.default_rng(5)
    sem = rng.integers(2, 8194, T).astype(np.uint32)
    ac = rng.integers(2, 23, (T, 36)).astype(np.uint32)
    for _ in range(warm):
        eng.codec_decode(sem, ac)
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        eng.codec_decode(sem, ac)
        times.append(time.perf_counter() - t)
    cms = float(np.median(times)) * 1000.0
    fl = codec_flops(T)
    codec = {"frames": T, "audio_s": T * 0.08, "ms": round(cms, 3),
             "x_realtime": round(T * 0.08 / (cms * 1e-3), 1),
             "algorithmic_GFLOP": round(fl / 1e9, 2),
             "TFLOPs": round(fl / (cms * 1e-3) / 1e12, 2),
             "mfma_issued_frac_of_peak": round(2 * fl / (cms * 1e-3) / 2.5e15, 4),
             "note": "wall time per call incl. code upload and audio readback, median of "
                     f"{reps} after {warm} warm-up calls; "
                     "f16 weights x hi/lo f16 activations on MFMA (2 issued flops per "
                     "algorithmic flop)"}
    log(f"[gpu] codec decode {T} frames: {cms:.2f} ms = {codec['x_realtime']:.0f}x real-time, "
        f"{codec['TFLOPs']:.1f} TFLOP/s algorithmic")
    return codec


STREAM_TBPS = 6.8  # a plain grid-stride read of 2 GiB with non-temporal loads on this part


def measure_timeline(eng, calls=20):
    """The held decode step (context 512) replayed from a graph in which every
    block of every launch records its start and end on the 100 MHz wall
    clock (vx_debug_timeline).  Per launch type: kernel time (earliest block
    start to latest block end), the boundary before it (previous launch's
    end to this launch's start), and the kernel time above a STREAM_TBPS
    stream of the launch's algorithmic bytes."""
    kinds = ["qkv", "attn_partial", "attn_combine", "oproj", "gateup", "down"]
    keys = eng.position + 1
    kv = 4 if eng.config.kv_f16 == 0 else 2
    algo = {"qkv": 37_748_736 + 2 * 1024 * kv, "attn_partial": keys * 2 * 1024 * kv,
            "attn_combine": 0, "oproj": 25_165_824, "gateup": 113_246_208, "down": 56_623_104,
            "final_norm": 0}
    busy = {k: [] for k in kinds + ["final_norm"]}
    gap = {k: [] for k in kinds + ["final_norm"]}
    spans = []
    eng.timeline(3)
    for _ in range(calls):
        ts = eng.timeline(2).astype(np.int64)
        n = ts.shape[0]
        spans.append((ts[-1, 1] - ts[0, 0]) / 100.0)
        for i in range(n):
            k = kinds[i % 6] if i < n - 1 else "final_norm"
            busy[k].append((ts[i, 1] - ts[i, 0]) / 100.0)
            if i > 0:
                gap[k].append((ts[i, 0] - ts[i - 1, 1]) / 100.0)
    L = eng.config.n_layers
    rows = {}
    tot_busy = tot_gap = tot_stream = 0.0
    for k in kinds + ["final_norm"]:
        per_step = L if k != "final_norm" else 1
        b = float(np.mean(busy[k]))
        g = float(np.mean(gap[k]))
        st = algo[k] / (STREAM_TBPS * 1e6)
        rows[k] = {"launches_per_step": per_step, "kernel_us": round(b, 3), "boundary_before_us": round(g, 3),
                   "stream_us": round(st, 3), "above_stream_us": round(b - st, 3)}
        tot_busy += b * per_step
        tot_gap += g * per_step
        tot_stream += st * per_step
    # the plain held step, graph-replayed without stamps, for comparison
    eng.time_backbone_steps(20, hold_position=True)
    plain = eng.time_backbone_steps(200, hold_position=True) / 200 * 1000
    return {"context_keys": keys, "calls": calls, "launches": int(6 * L + 1),
            "step_span_us": round(float(np.median(spans)), 2), "plain_step_us": round(plain, 2),
            "kernel_us": round(tot_busy, 1), "boundary_us": round(tot_gap, 1),
            "stream_us_at_%.1f_TBps" % STREAM_TBPS: round(tot_stream, 1),
            "kernel_above_stream_us": round(tot_busy - tot_stream, 1),
            "per_launch_type": rows,
            "note": "wall-clock stamps (100 MHz): every block of every launch stores its start and "
                    "end to its own slot (vector stores), in a copy of the held-step graph; kernel = "
                    "earliest block start to latest block end; boundary = gap between a launch's "
                    "latest block end and the next launch's earliest block start"}


def cpu_baseline(target_s):
    """The oracle (C restatement of the reference kernels, OpenMP) on the
    host.  value: full-depth 26-layer decode steps at context 512, no LM head
    (the headline unit).  frame_loop: whole frames at context 512 in the
    reference's dataflow (src/engine.ts:1020-1033, 1057-1225: the LM head
    every step, the flow-matching transformer per position and per guidance
    branch, 6 reads of every FM weight per Euler step) and in the optimal one
    (no LM head, positions and branches batched per weight read, as the GPU
    runs it); each a bounded sample of about target_s seconds."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle as O
    from vxtest import fill_oracle_kv
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    t0 = time.time()
    o = O.OracleEngine(O.default_config(), max_seq=CTX + 1)
    o.init_synthetic(0, 0.02)
    fill_oracle_kv(o, 0, CTX)
    log(f"[cpu] oracle ready in {time.time() - t0:.1f}s ({threads} threads)")
    x = O.gen_f32(0, "input.hidden", 3072)

    def sample(run, budget, cap=50, least=3):
        times = []
        while (sum(times) < budget and len(times) < cap) or len(times) < least:
            t = time.perf_counter()
            run()
            times.append(time.perf_counter() - t)
        return float(np.median(times[1:] if len(times) > 2 else times)), len(times)

    def step():
        o.position = CTX
        o.backbone_step(precomputed=x)
    med, n = sample(step, target_s)
    noise = O.gen_gauss_f32(0, "fm.noise", 36)
    table = o.weight("mm_audio_embeddings.audio_codebook_embeddings.embeddings.weight").reshape(-1, 3072)
    codes = np.full(36, 12, np.uint32)

    def frame(reference):
        o.position = CTX
        emb = O.multi_codebook_embed(table, 100, codes, 3072)
        o.backbone_step(precomputed=emb, lm_head=reference)
        o.fm_forward(noise, batched=not reference)
    fref, nref = sample(lambda: frame(True), target_s, least=2)
    fopt, nopt = sample(lambda: frame(False), target_s, least=2)
    o.close()
    log(f"[cpu] decode step {med * 1e3:.0f} ms; frame {fref * 1e3:.0f} ms (reference dataflow), "
        f"{fopt * 1e3:.0f} ms (optimal)")
    return {"value": 1.0 / med, "unit": "frames/s", "cores": threads, "kind": "port",
            "sample": f"{n} full 26-layer decode steps at context 512 (median of "
                      f"{max(1, n - 1)} after 1 warm-up), C oracle restating the "
                      f"reference WGSL kernels, OpenMP {threads} threads",
            "frame_loop": {
                "reference_dataflow": {"ms_per_frame": round(fref * 1e3, 1),
                                       "frames_per_s": round(1.0 / fref, 3),
                                       "x_realtime": round(0.08 / fref, 4), "frames_timed": nref},
                "optimal_dataflow": {"ms_per_frame": round(fopt * 1e3, 1),
                                     "frames_per_s": round(1.0 / fopt, 3),
                                     "x_realtime": round(0.08 / fopt, 4), "frames_timed": nopt},
                "sample": "whole frames at context 512 (multi-codebook embed, 26-layer step, "
                          "fmForward with 7 CFG Euler updates), median after 1 warm-up; reference "
                          "dataflow: LM head every step and the FM per position and branch "
                          "(src/engine.ts:1020-1033, 1057-1225); optimal: the GPU's dataflow"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--frames", type=int, default=500)
    ap.add_argument("--kernel-iters", type=int, default=104)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-frames", action="store_true")
    ap.add_argument("--no-f16-kv", action="store_true", help="skip the f16-KV-cache variant")
    ap.add_argument("--no-long", action="store_true", help="skip the context-4096 decode")
    ap.add_argument("--copy-probe-mb", type=int, default=0,
                    help="also run a plain device copy of this many MB (a known-traffic "
                         "kernel for scaling hardware byte counters)")
    ap.add_argument("--section", choices=["all", "codec", "prompt", "prefill", "timeline"], default="all",
                    help="codec: only the codec decoder measurement (a 1-layer engine), "
                         "printed as {\"codec\": ...}; prompt: only the 256-token prompt "
                         "(26 layers), printed as {\"prompt\": ...}; prefill: the same "
                         "without its decode steps; timeline: the launch timeline of the "
                         "headline decode step (26 layers, context 512), printed as "
                         "{\"timeline\": ...}")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the frame loop runs on a single MI355X "
              "(multi-GPU sharding is a design note, not a measured path); use --gpus 1",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_probe_mb:
        import torch
        n = args.copy_probe_mb * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
        log(f"[gpu] copy probe: 3 x {args.copy_probe_mb} MB device copy")

    import voxtral_amd as V
    if args.section == "codec":
        eng = V.VoxtralEngine(V.default_config(n_layers=1), max_seq_len=64).init()
        eng.init_synthetic(0, 0.02)
        print(json.dumps({"codec": measure_codec(eng)}), flush=True)
        eng.destroy()
        return
    if args.section in ("prompt", "prefill"):
        eng = V.VoxtralEngine(V.default_config(), max_seq_len=4096).init()
        eng.init_synthetic(0, 0.02)
        print(json.dumps({"prompt": measure_prompt(eng, decode=args.section == "prompt")}), flush=True)
        eng.destroy()
        return
    t0 = time.time()
    eng = prefilled_engine(V, kv_f16=False)
    log(f"[gpu] weights + {CTX}-token prefill in {time.time() - t0:.1f}s")
    if args.section == "timeline":
        tl = measure_timeline(eng)
        for k, r in tl["per_launch_type"].items():
            log(f"[gpu] {k:13s} kernel {r['kernel_us']:7.2f} us  boundary before {r['boundary_before_us']:5.2f} us  "
                f"above a {STREAM_TBPS} TB/s stream {r['above_stream_us']:6.2f} us")
        log(f"[gpu] step span {tl['step_span_us']} us (plain graph {tl['plain_step_us']} us): "
            f"kernels {tl['kernel_us']} us, boundaries {tl['boundary_us']} us")
        print(json.dumps({"timeline": tl}), flush=True)
        eng.destroy()
        return

    # ---- headline: decode steps at context 512 (513 keys each)
    eng.time_backbone_steps(args.warmup, hold_position=True)
    ms = eng.time_backbone_steps(args.steps, hold_position=True)
    ms_step = ms / args.steps
    value = 1000.0 / ms_step
    sb = step_bytes(CTX + 1)
    step_gbps = sb / (ms_step * 1e-3) / 1e9
    log(f"[gpu] decode {ms_step * 1000:.1f} us/step -> {value:.1f} frames/s, "
        f"{step_gbps:.0f} GB/s ({step_gbps / HBM_PEAK_GBPS:.1%} of peak)")

    # ---- dominant kernel: gate/up GEMV (+RMSNorm prologue, SwiGLU epilogue)
    kern = {}
    for k, name in enumerate(V.KERNEL_NAMES):
        us, b = eng.time_kernel(k, args.kernel_iters)
        kern[name] = {"avg_us": us, "bytes": b, "GBps": b / (us * 1e-6) / 1e9}
        log(f"[gpu] kernel {name:7s} {us:8.2f} us  {b / 1e6:8.2f} MB  {kern[name]['GBps']:7.0f} GB/s")
    dom = kern["gateup"]
    # achieved / frac on the kernel-trace average of the committed rocprofv3
    # summary (eager launches; per-dispatch durations), the live HIP-event
    # average beside it (back-to-back launches on the engine's stream)
    t_us = trace_avg_us("gateup")
    us = t_us if t_us is not None else dom["avg_us"]
    gbps = dom["bytes"] / (us * 1e-6) / 1e9
    roofline = {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(gbps / HBM_PEAK_GBPS, 4),
                "traffic": measured_traffic("gateup"),
                "kernel": "gemv1_kernel<gate/up + RMSNorm + SwiGLU>", "launch_bytes": dom["bytes"],
                "avg_us_trace": t_us, "avg_us_events": round(dom["avg_us"], 3),
                "achieved_events": round(dom["GBps"], 1),
                "frac_events": round(dom["GBps"] / HBM_PEAK_GBPS, 4),
                "basis": "trace" if t_us is not None else "events"}

    # ---- full frame loop (backbone + FM CFG Euler loop), 500 frames
    frame = None
    if not args.no_frames:
        eng.position = CTX
        eng.debug_write("normed", np.zeros(3072, np.float32))
        eng.fm_step_and_read()  # seeds the device codes read by the first frame
        eng.time_frames(5)
        eng.position = CTX
        fms = eng.time_frames(args.frames)
        fps = args.frames * 1000.0 / fms
        keys_avg = CTX + 1 + (args.frames - 1) / 2.0
        fb = step_bytes(keys_avg) + 7 * FM_EULER_BYTES + FM_FRAME_BYTES + EMB_CODES_BYTES
        frame = {"frames": args.frames, "ms_per_frame": round(fms / args.frames, 4),
                 "frames_per_s": round(fps, 2), "x_realtime": round(fps * 0.08, 2),
                 "bytes_per_frame": fb,
                 "hbm_frac": round(fb * fps / 1e9 / HBM_PEAK_GBPS, 4),
                 "sampling": "greedy masked argmax on device, no EOS",
                 "launches_per_euler_step": 16}
        log(f"[gpu] frame loop {fms / args.frames * 1000:.1f} us/frame -> {fps:.1f} frames/s "
            f"= {fps * 0.08:.1f}x real-time")

    # ---- the flow-matching kernels one by one (after the frame loop, on the
    # buffers a frame leaves), cycling over the 3 FM layers
    fm_kern = None
    if not args.no_frames:
        fm_kern = {}
        for k, name in enumerate(V.FM_KERNEL_NAMES):
            us, b = eng.time_kernel(len(V.KERNEL_NAMES) + k, 63)
            gbps = b / (us * 1e-6) / 1e9
            fm_kern[name] = {"avg_us": round(us, 3), "bytes": b, "GBps": round(gbps, 1),
                             "frac": round(gbps / HBM_PEAK_GBPS, 4)}
            log(f"[gpu] kernel {name:10s} {us:8.2f} us  {b / 1e6:8.2f} MB  {gbps:7.0f} GB/s")

    # ---- the 256-token prompt + 500 frame steps (the reference prefills per token)
    prompt = None
    if not args.no_long:
        prompt = measure_prompt(eng)
        log(f"[gpu] prompt: prefill 256 tokens in {prompt['prefill_ms']:.2f} ms "
            f"({prompt['mfma_issued_TFLOPs']:.0f} TFLOP/s issued, "
            f"{prompt['mfma_frac_of_peak']:.1%} of MFMA peak); 500 decode steps "
            f"{prompt['decode_frames_per_s']:.1f} frames/s")

    # ---- generate() end to end (prompt, kick, 200 frames, callbacks), per sampling mode
    gen = None
    if not args.no_long:
        gen = {}
        toks = list(np.random.default_rng(3).integers(0, 131072, 64))
        for mode in ("top_p", "top_p_host", "greedy"):
            eng.generate(toks, 0, 0, None, 8, sampling=mode, seed=1, ignore_eos=True)
            t = time.perf_counter()
            r = eng.generate(toks, 0, 0, None, 200, sampling=mode, seed=1, ignore_eos=True)
            dt = time.perf_counter() - t
            fr = r["stats"]["framesGenerated"]
            gen[mode] = {"frames": fr, "s": round(dt, 4), "frames_per_s": round(fr / dt, 2),
                         "x_realtime": round(fr / dt * 0.08, 2),
                         "codec_ms": round(r["stats"]["codecMs"], 3),
                         "audio_samples": int(r["audio"].size)}
            log(f"[gpu] generate({mode}): {fr} frames in {dt * 1000:.0f} ms -> "
                f"{fr / dt:.1f} frames/s = {fr / dt * 0.08:.1f}x real-time")

    # ---- codec decoder: 250 frames (20 s of audio) of random codes
    codec = None if args.no_long else measure_codec(eng)

    # ---- long-context decode: 200 steps at positions 3896..4095 over a
    # synthetic N(0,1) KV cache (values f16-exact), context growing to 4096
    long_ctx = None
    if not args.no_long:
        start, n = 3896, 200
        eng.fill_kv_synthetic(0, start)
        eng.position = start
        eng.time_backbone_steps(5, hold_position=True)
        lms = eng.time_backbone_steps(n, hold_position=False)
        lfps = n * 1000.0 / lms
        lb = step_bytes(start + 1 + (n - 1) / 2.0)
        long_ctx = {"positions": [start, start + n - 1], "steps": n,
                    "ms_per_step": round(lms / n, 5), "frames_per_s": round(lfps, 2),
                    "hbm_frac": round(lb * lfps / 1e9 / HBM_PEAK_GBPS, 4)}
        log(f"[gpu] context {start}..{start + n}: {lms / n * 1000:.1f} us/step -> {lfps:.1f} frames/s")

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"[cpu] {cpu['value']:.3f} frames/s on {cpu['cores']} threads")

    # the f16-KV engine is created while the first one still holds its
    # memory: device memory released just before (hipFree of ~9 GB) slows HBM
    # streaming by a few percent for a second or more while the driver takes
    # it back, which would be charged to the variant
    f16kv = None
    if not args.no_f16_kv:
        e16 = prefilled_engine(V, kv_f16=True)
        e16.time_backbone_steps(args.warmup, hold_position=True)
        ms16 = e16.time_backbone_steps(args.steps, hold_position=True) / args.steps
        b16 = step_bytes(CTX + 1, 2)
        f16kv = {"frames_per_s": round(1000.0 / ms16, 2), "ms_per_step": round(ms16, 5),
                 "step_hbm_frac": round(b16 / (ms16 * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
                 "note": "optional f16 KV cache; held to the 1e-2 bar against the oracle's f16-KV mode at 26 layers "
                         "(positions 3896-3899 over an N(0,1) cache)"}
        log(f"[gpu] f16 KV cache: {ms16 * 1000:.1f} us/step -> {1000.0 / ms16:.1f} frames/s")
        if not args.no_long:
            # the long-context stress with the f16 N(0,1) cache it is specified with
            start, n = 3896, 200
            e16.fill_kv_synthetic(0, start)
            e16.position = start
            e16.time_backbone_steps(5, hold_position=True)
            lms = e16.time_backbone_steps(n, hold_position=False)
            lfps = n * 1000.0 / lms
            lb = step_bytes(start + 1 + (n - 1) / 2.0, 2)
            f16kv["long_context"] = {"positions": [start, start + n - 1], "steps": n,
                                     "ms_per_step": round(lms / n, 5), "frames_per_s": round(lfps, 2),
                                     "hbm_frac": round(lb * lfps / 1e9 / HBM_PEAK_GBPS, 4)}
            log(f"[gpu] f16 KV cache, context {start}..{start + n}: {lms / n * 1000:.1f} us/step "
                f"-> {lfps:.1f} frames/s")
        e16.destroy()
    eng.destroy()

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "frames/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "weights_dtype": "f16", "kv_dtype": "f32", "data": "synthetic",
        "config": {"workload": "26-layer backbone decode, batch 1, context 512 (513 keys), "
                               "after a real 512-token prefill", "layers": LAYERS,
                   "context": CTX, "batch": 1, "parallelism": "none (1 GPU)"},
        "step_hbm": {"bytes": sb, "achieved_GBps": round(step_gbps, 1),
                     "frac": round(step_gbps / HBM_PEAK_GBPS, 4)},
        "roofline": roofline, "kernels": {k: {kk: round(vv, 3) for kk, vv in v.items()}
                                          for k, v in kern.items()},
        "frame_loop": frame, "fm_kernels": fm_kern, "generate": gen, "prompt": prompt, "codec": codec,
        "long_context": long_ctx,
        "f16_kv_variant": f16kv,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
