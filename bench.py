#!/usr/bin/env python3
"""Benchmark of the MI355X decode path: codec frames/s, batch 1, at KV 2048.

Workload (one "step" = one frame): the full 28-layer Talker (hidden 2048,
16/8 heads, FFN 6144, codec vocab 3072) plus the 5-layer code predictor
(15 codebooks), random Q4 weights, a synthetic prompt of 64 text ids
(uniform in [0, 151936)) embedded through the text projection and
prefilled at positions 0..63, then the frame loop with top-k 50,
temperature 0.9, repetition penalty 1.05, seed 42, EOS disabled (random
weights can emit it).  The loop runs untimed from KV 64 to KV 2048 (the
last --warmup of those frames are the warm-up), then --steps frames are
timed from KV 2048 (64 steps: KV 2048 -> 2112, the last frames of the
2048-frame workload).  The whole loop's average from KV 64 is reported
beside it.

Printed as one JSON line: frames/s over the timed frames (whole job, inputs
resident in HBM); the roofline of the Q4 GEMV k=2048 -> n=6144 on a rotating
pool of 64 weights (HIP events around back-to-back launches), with a
streaming read of the same bytes as its attainable single-launch bound; the
same GEMV kernel streaming a 113 MB weight; the talker gate|up and attention
kernels and a float4 copy; and the oracle's CPU frame rate on a bounded
sample at KV 2048 as the CPU baseline.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qora-tts-12hz-1.7b_amd"))

HBM_PEAK_GBS = 8000.0
F32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense f32 matrix peak
F16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix peak
ICL_ROWS = 400                 # ICL prompt positions (text + reference codes)
TTS_PAD = 151671          # generate_new.rs:28
PROMPT = 64                    # prompt positions
KV_HEADLINE = 2048             # KV length the headline frames start from


# The standalone GEMV's kernel instance (tile G1_T256: one 32-column group x
# 2048 rows per workgroup, plain prologue, partial epilogue); no frame stage
# uses this instance, so rocprof's line for it covers exactly the GEMV
# timing launches.
GEMV_KERNEL = "k_gemv<256, 1, 8, 1, ProPlain<1>, EpiPart<1>>"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "q4_gemv_2048x6144_hbm_traffic.txt")


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel factor), or
    None when that summary is absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1])), os.path.relpath(TRAFFIC_FILE, ROOT)
    except OSError:
        pass
    return None, None


FUSED_FILE = os.path.join(ROOT, "profiles", "frame_fused_kernels_traffic.txt")


def fused_profile():
    """Per-launch rows of the committed profile of the frame's fused
    launches (kernel trace + FETCH_SIZE / WRITE_SIZE / L2 counter passes of
    bench.py --fused-only): {description: {avg_us, alg_bytes, counter_bytes,
    ratio, frac, l2_hit}}, or {} when the summary is absent."""
    rows = {}
    try:
        with open(FUSED_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) < 11 or not parts[-1].replace(".", "").isdigit():
                    continue
                try:
                    n, avg, med = int(parts[-9]), float(parts[-8]), float(parts[-7])
                    alg, cb = int(parts[-6].replace(",", "")), int(parts[-5].replace(",", ""))
                    ratio, gbs, frac, l2 = (float(x) for x in parts[-4:])
                except ValueError:
                    continue
                desc = " ".join(parts[:-9])
                rows[desc] = {"dispatches": n, "avg_us": avg, "median_us": med, "alg_bytes": alg,
                              "counter_bytes": cb, "traffic_ratio": ratio, "alg_gbs": gbs, "frac": frac,
                              "l2_hit": l2}
    except OSError:
        pass
    return rows


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# Decode GEMV shapes (k -> n, fused as the frame runs them) for the per-shape
# sweep of the standalone Q4 GEMV.
SWEEP_SHAPES = [("talker q|k|v", 2048, 4096), ("talker o", 2048, 2048), ("talker gate|up", 2048, 12288),
                ("talker down", 6144, 2048), ("codec head", 2048, 3072), ("predictor q|k|v", 1024, 4096),
                ("predictor gate|up", 1024, 6144), ("predictor down", 3072, 1024), ("predictor head", 1024, 2048)]


def gemv_sweep(ctx, synth, pool_bytes=320 << 20):
    """Standalone Q4 GEMV GB/s on each decode shape, cycling a pool of device
    copies larger than the 256 MB last-level cache."""
    rng = np.random.Generator(np.random.PCG64(5))
    out = {}
    for name, k, n in SWEEP_SHAPES:
        w = synth.q4_random(rng, k, n)
        copies = max(8, -(-pool_bytes // int(k * n * 0.5625)))
        pool = [ctx.upload(w) for _ in range(copies)]
        us, b = ctx.time_gemv(pool, 4 * copies)
        for d in pool:
            d.free()
        out[f"{name} {k}x{n}"] = {"us": round(us, 2), "gbs": round(b / us / 1e3, 1),
                                   "frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4)}
    return out


def host_info():
    model, flags = "unknown", set()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name") and model == "unknown":
                    model = line.split(":", 1)[1].strip()
                elif line.startswith("flags") and not flags:
                    flags = set(line.split(":", 1)[1].split())
    except OSError:
        pass
    isa = "avx512f" if "avx512f" in flags else ("avx2" if "avx2" in flags else "other")
    return {"cpu": model, "nproc": os.cpu_count(), "isa": isa}


def cpu_gemv(seconds=3.0):
    """The oracle's restatement of gemv_q4 (chunk/pool policy) on the
    2048 x 6144 GEMV: min(nproc, 16) workers and one thread, with the inner
    kernel the reference picks on this host (gemv.rs:230-243: AVX-512 when
    present) and with the AVX2 kernel beside it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from qtts import synth
    rng = np.random.Generator(np.random.PCG64(1))
    w = synth.q4_random(rng, 2048, 6144)
    x = rng.standard_normal(2048).astype(np.float32)
    nbytes = 2048 * 6144 * 0.5625 + 4 * 2048 + 4 * 6144
    res = {}
    isas = [oracle.set_isa(None)]
    if isas[0] != "avx2" and oracle.set_isa("avx2"):
        isas.append("avx2")
    for isa in isas:
        oracle.set_isa(None if isa == isas[0] else isa)
        for label, workers in (("pool", min(os.cpu_count() or 1, 16)), ("one_thread", 1)):
            oracle.set_workers(workers, workers)
            oracle.gemv(x, w)
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < seconds / (2 * len(isas)):
                oracle.gemv(x, w)
                n += 1
            us = (time.perf_counter() - t0) / n * 1e6
            key = label if isa == isas[0] else f"{label}_{isa}"
            res[key] = {"threads": workers, "isa": isa, "us": round(us, 1), "gbs": round(nbytes / us / 1e3, 2)}
    oracle.set_isa(None)
    return res


def cpu_baseline(talker, pred, logits, hidden, pad, kv_len, seconds, isa=None):
    """Oracle (C restatement of the reference's CPU path, gemv pool of
    min(nproc, 16) workers, the inner GEMV kernel the reference picks on this
    host or `isa`) timed on a bounded sample: frames at KV ~kv_len after a
    synthetic N(0,1) KV prefill."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    import qtts
    workers = min(os.cpu_count() or 1, 16)
    oracle.set_workers(workers, workers)
    used_isa = oracle.set_isa(isa)
    om = oracle.Model(talker, pred, kv_cap=kv_len + 64)
    rng = np.random.Generator(np.random.PCG64(7))
    L = len(talker.layers)
    K = rng.standard_normal((L, kv_len, 8, 128), dtype=np.float32)
    V = rng.standard_normal((L, kv_len, 8, 128), dtype=np.float32)
    om.kv_load(K, V)
    del K, V
    params = qtts.sample_params(eos_enabled=False)
    om.gen_begin(logits, hidden, kv_len, 42)
    n = 0
    t0 = time.perf_counter()
    while True:
        om.frame(params, pad)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 64:
            break
    om.close()
    oracle.set_isa(None)
    return {"value": n / el, "unit": "frames/s", "cores": workers, "kind": "port", "isa": used_isa,
            "sample": f"{n} frames of the 28-layer talker + 5-layer predictor at KV {kv_len}..{kv_len + n} "
                      f"(synthetic N(0,1) KV prefill), {el:.1f} s, {used_isa} GEMV kernel"}


def time_prefill(ctx, layers):
    """The ICL-prompt prefill on the matrix cores: the gate|up GEMM alone
    (cycling the layers) and the whole 400-position prefill, as achieved
    TFLOP/s of the algorithmic (f32-accurate) work.  The GEMMs issue that
    work as three f16 matrix products per pair of split operands
    (QTTS_GEMM_F32=1: f32 matrix instructions instead), so `mfma_issue_frac`
    is the issued rate (3x the algorithmic one) against the dense f16 MFMA
    peak, and `over_f32_mfma_peak` compares the algorithmic rate with what
    f32 matrix instructions could reach at most (above 1 on the f16 path)."""
    f32 = os.environ.get("QTTS_GEMM_F32", "0") not in ("", "0")
    issue, peak = (1, F32_MFMA_PEAK_TFLOPS) if f32 else (3, F16_MFMA_PEAK_TFLOPS)
    g_us, g_fl = ctx.time_prefill(ICL_ROWS, 0, 4 * layers)
    p_us, p_fl = ctx.time_prefill(ICL_ROWS, 1, 3)
    g_tf, p_tf = g_fl / g_us / 1e6, p_fl / p_us / 1e6
    log(f"prefill {ICL_ROWS} rows: {p_us / 1e3:.2f} ms ({p_tf:.1f} TFLOP/s); gate|up GEMM {g_us:.1f} us "
        f"({g_tf:.1f} TFLOP/s = {g_tf / F32_MFMA_PEAK_TFLOPS:.2f}x the f32 MFMA peak; "
        f"matrix instructions issued at {issue * g_tf / peak:.1%} of their peak)")
    return {"rows": ICL_ROWS, "ms": round(p_us / 1e3, 3), "tflops": round(p_tf, 2),
            "over_f32_mfma_peak": round(p_tf / F32_MFMA_PEAK_TFLOPS, 4), "flops": p_fl,
            "gate_up_gemm": {"shape": f"[{ICL_ROWS} x 2048] x [2048 x 12288], SwiGLU epilogue", "us": round(g_us, 2),
                             "tflops": round(g_tf, 2), "over_f32_mfma_peak": round(g_tf / F32_MFMA_PEAK_TFLOPS, 4),
                             "mfma_issue_frac": round(issue * g_tf / peak, 4), "flops": g_fl},
            "f32_mfma_peak_tflops": F32_MFMA_PEAK_TFLOPS, "issue_peak_tflops": peak,
            "dtype": "f32 (v_mfma_f32_16x16x4_f32)" if f32 else
                     "f32-accurate: operands split into f16 hi + lo, hi*hi + hi*lo + lo*hi on "
                     "v_mfma_f32_16x16x32_f16 with f32 accumulation"}


ICL_FRAMES = 512               # decode frames after the ICL prompt (KV 400 -> 912)
TALKER_FRAME_BYTES = 796_262_400 + 247_808   # 28 layers of Q4 weights + codec head, gammas
PRED_FRAME_BYTES = 63_111_168                # predictor weights, each read once (unique bytes)
KV_BYTES_PER_POS = 229_376                   # K + V, 28 layers x 8 heads x 128 x f32 x 2


def frame_bytes(kv_len):
    """Algorithmic HBM bytes of one frame at KV length L: weights once, L
    cached positions read, one written."""
    return TALKER_FRAME_BYTES + PRED_FRAME_BYTES + KV_BYTES_PER_POS * (kv_len + 1)


def time_icl_decode(ctx, params, pad):
    """The ICL workload: a 400-position prompt built on the device from
    reference ids, text ids and 16 x 399 reference codes
    (build_icl_block), prefilled, then ICL_FRAMES frames (KV 400 -> 912)."""
    rng = np.random.Generator(np.random.PCG64(5))
    n_ref, n_text, n_codes = 100, 200, ICL_ROWS - 1
    ref = rng.integers(0, 151936, n_ref)
    text = rng.integers(0, 151936, n_text)
    codes = rng.integers(0, 2048, (16, n_codes))
    ctx.kv_reset()
    ctx.lib.qtts_sync(ctx.h)
    t0 = time.perf_counter()
    icl, rem = ctx.build_icl_block(ref, text, codes)
    hidden = ctx.prefill_talker_raw_from(icl, 0)
    logits = ctx.apply_codec_head(hidden)
    t_prompt = time.perf_counter() - t0
    ctx.gen_set_text(rem if len(rem) else None, pad)
    ctx.gen_begin(logits, hidden, len(icl), 42, params)
    ctx.lib.qtts_sync(ctx.h)
    t0 = time.perf_counter()
    out, _ = ctx.gen_frames(ICL_FRAMES)
    ctx.lib.qtts_sync(ctx.h)
    dt = time.perf_counter() - t0
    n = out.shape[0]
    log(f"ICL prompt {len(icl)} rows built + prefilled in {t_prompt * 1e3:.1f} ms; {n} frames at KV {len(icl)} -> "
        f"{len(icl) + n}: {n / dt:.1f} frames/s")
    return {"prompt_rows": len(icl), "prompt_ms": round(t_prompt * 1e3, 2),
            "prompt_note": "build_icl_block + prefill + codec head, rows staged through host memory",
            "frames": n, "kv_start": len(icl), "kv_end": len(icl) + n, "frames_per_s": round(n / dt, 2)}


DEC_FRAMES = 160               # speech-decoder workload: 160 codec frames = 12.8 s of 24 kHz audio
DEC_RATE = 24000


def time_decoder(synth, qtts, cpu_frames=0):
    """decode_to_audio on the device (the 12 Hz tokenizer's decoder shapes,
    random f32 weights) over DEC_FRAMES synthetic frames: audio seconds per
    second and achieved TFLOP/s of the algorithmic (f32-accurate) work; the
    convolution GEMMs issue it as three f16 matrix products per pair of split
    operands (QTTS_DEC_F32=1: f32 matrix instructions), so `mfma_issue_frac`
    is the issued rate against that instruction's peak (the decode's few
    FLOPs outside the GEMMs counted as GEMM work).  With cpu_frames, the
    oracle's C decoder on that many frames (all host threads) beside it."""
    f32 = os.environ.get("QTTS_DEC_F32", "0") not in ("", "0")
    issue, peak = (1, F32_MFMA_PEAK_TFLOPS) if f32 else (3, F16_MFMA_PEAK_TFLOPS)
    d = synth.make_decoder(seed=7)
    ctx = qtts.Context(0, kv_capacity=64)
    ctx.upload_decoder(d)
    us, fl = ctx.time_decode(DEC_FRAMES, 5)
    ctx.close()
    audio_s = DEC_FRAMES * d.upsample_factor / DEC_RATE
    tf = fl / us / 1e6
    log(f"speech decoder {DEC_FRAMES} frames: {us / 1e3:.2f} ms, {audio_s / (us * 1e-6):.0f} audio s/s, "
        f"{tf:.1f} TFLOP/s ({tf / F32_MFMA_PEAK_TFLOPS:.2f}x the f32 MFMA peak)")
    out = {"frames": DEC_FRAMES, "samples": DEC_FRAMES * d.upsample_factor, "ms": round(us / 1e3, 3),
           "audio_seconds_per_second": round(audio_s / (us * 1e-6), 1), "frames_per_second": round(DEC_FRAMES / (us * 1e-6), 1),
           "tflops": round(tf, 2), "over_f32_mfma_peak": round(tf / F32_MFMA_PEAK_TFLOPS, 4),
           "mfma_issue_frac": round(issue * tf / peak, 4), "flops": fl,
           "f32_mfma_peak_tflops": F32_MFMA_PEAK_TFLOPS, "issue_peak_tflops": peak,
           "dtype": "f32 (v_mfma_f32_16x16x4_f32)" if f32 else
                    "f32-accurate: convolution GEMM operands split into f16 hi + lo on v_mfma_f32_16x16x32_f16, "
                    "f32 accumulation"}
    if cpu_frames:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O
        threads = min(os.cpu_count() or 1, 16)
        codes = np.random.Generator(np.random.PCG64(5)).integers(0, 2048, (16, cpu_frames)).astype(np.uint32)
        t0 = time.perf_counter()
        O.decode_to_audio(d, codes, threads=threads)
        el = time.perf_counter() - t0
        out["cpu_baseline"] = {"value": round(cpu_frames * d.upsample_factor / DEC_RATE / el, 3),
                               "unit": "audio s/s", "cores": threads, "kind": "port",
                               "sample": f"oracle decode of {cpu_frames} frames, {el:.1f} s"}
        log(f"cpu speech decoder: {out['cpu_baseline']['value']} audio s/s on {threads} threads")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64, help=f"timed frames from KV {KV_HEADLINE}")
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gemv-copies", type=int, default=64)
    ap.add_argument("--no-stream", action="store_true", help="skip the Q4 GEMV on a 2048 x 98304 weight")
    ap.add_argument("--prefill-only", action="store_true", help="time only the matrix-core prefill")
    ap.add_argument("--no-sweep", action="store_true", help="skip the per-shape GEMV sweep")
    ap.add_argument("--decoder-only", action="store_true", help="time only the speech decoder")
    ap.add_argument("--no-decoder", action="store_true", help="skip the speech decoder")
    ap.add_argument("--no-icl", action="store_true", help="skip the ICL workload (400-row prompt + 512 frames)")
    ap.add_argument("--attention-only", action="store_true",
                    help="time only the talker decode attention at KV 2048 (and the copy calibration)")
    ap.add_argument("--frames-only", action="store_true",
                    help=f"only --steps frames from KV {KV_HEADLINE}, the cache filled by a prefill of N(0,1) rows "
                         f"(for kernel profiles of the frame at the headline KV)")
    ap.add_argument("--frames-kv", type=int, default=KV_HEADLINE,
                    help=f"--frames-only: the cached positions the frames start from (default {KV_HEADLINE})")
    ap.add_argument("--fused-only", action="store_true",
                    help="only the frame's fused launches, standalone: one talker layer at KV 2048 (q|k|v + "
                         "attention, o-proj, gate|up + down) and one predictor layer step (q|k|v + attention + "
                         "o-proj, gate|up + down), cycling the layers, and the copy calibration (for counter passes)")
    ap.add_argument("--gemv-only", action="store_true",
                    help="only the Q4 GEMV 2048 x 6144 over its weight pool, the same-bytes streaming read "
                         "and the float4 copy (the counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported "
              f"(one utterance's decode is a serial chain; independent text chunks would each take one GPU)", file=sys.stderr)
        sys.exit(2)

    if args.steps < 1 or KV_HEADLINE + args.steps > 8192:
        print(f"--steps must be in 1..{8192 - KV_HEADLINE} (the cache holds 8192 positions)", file=sys.stderr)
        sys.exit(2)

    import qtts
    from qtts import synth

    if args.decoder_only:
        print(json.dumps({"speech_decoder": time_decoder(synth, qtts)}), flush=True)
        return

    t_gen = time.time()
    talker = synth.make_talker(seed=1, n_layers=args.layers)
    pred = synth.make_predictor(seed=2)
    log(f"synthetic model generated in {time.time() - t_gen:.1f}s")

    if not 1 <= args.frames_kv <= 8192 - args.steps - args.warmup:
        print(f"--frames-kv {args.frames_kv}: the cache holds at most 8192 positions", file=sys.stderr)
        sys.exit(2)
    cap = min(8192, -(-(max(KV_HEADLINE, args.frames_kv) + args.steps + args.warmup) // 64) * 64)
    ctx = qtts.Context(0, kv_capacity=max(cap, 4096))
    t_up = time.time()
    ctx.upload_model(talker, pred)
    log(f"uploaded in {time.time() - t_up:.1f}s")
    # what the model holds on the device; the predictor's upload-time tables
    # (projected code rows and their layer-0 q|k|v) are read one row per step
    mem = {k: round(v / 2**20, 1) for k, v in ctx.device_bytes().items()}
    if args.prefill_only:
        pf = time_prefill(ctx, args.layers)
        ctx.close()
        print(json.dumps({"prefill": pf}), flush=True)
        return
    if args.attention_only:
        # 2048 cached positions from a prefill of N(0,1) rows, then one decode
        # step's attention per layer (appending at 2048, attending 2049)
        X = np.random.Generator(np.random.PCG64(7)).standard_normal((2048, talker.hidden)).astype(np.float32)
        ctx.prefill_talker_raw_from(X, 0)
        a_us, a_bytes = ctx.time_kernel(1, 4 * args.layers)
        c_us, c_bytes = ctx.time_kernel(2, 20)
        ctx.close()
        print(json.dumps({"talker_attention": {"kv": 2049, "us": round(a_us, 2), "bytes": int(a_bytes),
                                               "gbs": round(a_bytes / a_us / 1e3, 1)},
                          "float4_copy_256MiB": {"us": round(c_us, 2), "gbs": round(c_bytes / c_us / 1e3, 1)}}),
              flush=True)
        return

    if args.fused_only:
        # 2048 cached positions from a prefill of N(0,1) rows; the talker
        # layer appends at 2048 and attends 2049, as the frame at KV 2048
        X = np.random.Generator(np.random.PCG64(7)).standard_normal((2048, talker.hidden)).astype(np.float32)
        ctx.prefill_talker_raw_from(X, 0)
        del X
        tl_us, tl_bytes = ctx.time_kernel(8, 4 * args.layers)
        pl_us, pl_bytes = ctx.time_kernel(9, 4 * 5 * 14)
        c_us, c_bytes = ctx.time_kernel(2, 20)
        ctx.close()
        print(json.dumps({"talker_layer_kv2049": {"launches": 3, "us": round(tl_us, 2), "bytes": int(tl_bytes),
                                                  "gbs": round(tl_bytes / tl_us / 1e3, 1)},
                          "predictor_layer_step": {"launches": 2, "us": round(pl_us, 2), "bytes": int(pl_bytes),
                                                   "gbs": round(pl_bytes / pl_us / 1e3, 1)},
                          "float4_copy_256MiB": {"us": round(c_us, 2), "gbs": round(c_bytes / c_us / 1e3, 1)}}),
              flush=True)
        return

    if args.gemv_only:
        grng = np.random.Generator(np.random.PCG64(1))
        pool = [ctx.upload(synth.q4_random(grng, 2048, 6144)) for _ in range(args.gemv_copies)]
        g_us, g_bytes = ctx.time_gemv(pool, 4 * args.gemv_copies)
        for w in pool:
            w.free()
        r_us, r_bytes = ctx.time_kernel(7, 256)
        c_us, c_bytes = ctx.time_kernel(2, 20)
        ctx.close()
        print(json.dumps({"q4_gemv_2048x6144": {"us": round(g_us, 3), "gbs": round(g_bytes / g_us / 1e3, 1)},
                          "read_same_bytes": {"us": round(r_us, 3), "gbs": round(r_bytes / r_us / 1e3, 1)},
                          "float4_copy_256MiB": {"us": round(c_us, 2), "gbs": round(c_bytes / c_us / 1e3, 1)}}),
              flush=True)
        return
    if args.frames_only:
        kv = args.frames_kv
        X = np.random.Generator(np.random.PCG64(7)).standard_normal((kv, talker.hidden)).astype(np.float32)
        hid = ctx.prefill_talker_raw_from(X, 0)
        del X
        pad = ctx.embed_text_token(TTS_PAD)
        ctx.gen_set_text(None, pad)
        ctx.gen_begin(ctx.apply_codec_head(hid), hid, kv, 42, qtts.sample_params(eos_enabled=False))
        ctx.gen_frames(args.warmup)
        ctx.lib.qtts_sync(ctx.h)
        t0 = time.perf_counter()
        codes, _ = ctx.gen_frames(args.steps)
        ctx.lib.qtts_sync(ctx.h)
        dt = time.perf_counter() - t0
        kv0 = kv + args.warmup
        ctx.close()
        print(json.dumps({"frames": codes.shape[0], "kv_start": kv0, "kv_end": kv0 + codes.shape[0],
                          "frames_per_s": round(codes.shape[0] / dt, 2)}), flush=True)
        return

    rng = np.random.Generator(np.random.PCG64(42))
    ids = rng.integers(0, 151936, PROMPT)
    prompt = np.stack([ctx.embed_text_token(int(i)) for i in ids])
    pad = ctx.embed_text_token(TTS_PAD)
    ctx.gen_set_text(None, pad)
    hidden = ctx.prefill_talker_raw_from(prompt, 0)
    logits = ctx.apply_codec_head(hidden)
    params = qtts.sample_params(eos_enabled=False)
    log(f"prefill done ({PROMPT} positions)")

    # the frame loop from KV 64: untimed up to KV 2048 (its last --warmup
    # frames are the warm-up), then --steps timed frames from KV 2048
    warm = min(args.warmup, KV_HEADLINE - PROMPT)
    ramp = KV_HEADLINE - PROMPT - warm
    ctx.gen_begin(logits, hidden, PROMPT, 42, params)
    ctx.lib.qtts_sync(ctx.h)
    t_ramp = time.perf_counter()
    done, _ = ctx.gen_frames(ramp)
    ctx.lib.qtts_sync(ctx.h)
    t_ramp = time.perf_counter() - t_ramp
    t_warm = time.perf_counter()
    done2, _ = ctx.gen_frames(warm)
    ctx.lib.qtts_sync(ctx.h)
    t_warm = time.perf_counter() - t_warm
    kv_start = ctx.kv_len()
    assert kv_start == KV_HEADLINE and done.shape[0] + done2.shape[0] == KV_HEADLINE - PROMPT, kv_start
    log(f"frames KV {PROMPT} -> {kv_start}: {(ramp + warm) / (t_ramp + t_warm):.1f} frames/s")

    t0 = time.perf_counter()
    codes, eos = ctx.gen_frames(args.steps)
    ctx.lib.qtts_sync(ctx.h)
    dt = time.perf_counter() - t0
    frames = codes.shape[0]
    fps = frames / dt
    log(f"{frames} frames in {dt:.4f}s -> {fps:.1f} frames/s (KV {kv_start} -> {kv_start + frames})")
    loop_frames = ramp + warm + frames
    loop = {"kv_start": PROMPT, "kv_end": kv_start + frames, "frames": loop_frames,
            "frames_per_s": round(loop_frames / (t_ramp + t_warm + dt), 2),
            "note": "the whole frame loop from the prompt, untimed ramp + warm-up + the timed frames"}

    # the frame's two halves, each captured alone and replayed (the state is
    # restored afterwards): the talker step at KV ~2112, and the sampler +
    # predictor chain + combine
    tk_us, tk_bytes = ctx.time_kernel(6, 16)
    pc_us, pc_bytes = ctx.time_kernel(5, 16)
    log(f"talker step {tk_us:.1f}us, sampler + predictor chain + combine {pc_us:.1f}us")
    split = {"talker_step_us": round(tk_us, 1), "talker_step_weight_bytes": int(tk_bytes),
             "predictor_chain_us": round(pc_us, 1), "predictor_weight_bytes": int(pc_bytes),
             "note": "each half of the frame captured alone and replayed back to back (KV ~2112); "
                     "the whole frame is slower than the sum by the predictor weights falling out "
                     "of the last-level cache between frames"}

    # kernels at the final KV length (~2112): HIP events around back-to-back
    # launches.  These two are the component kernels timed alone: in the frame
    # the attention shares a launch with the q|k|v GEMV, and the gate|up one
    # with the down projection.
    gu_us, gu_bytes = ctx.time_kernel(0, 4 * args.layers)
    at_us, at_bytes = ctx.time_kernel(1, 4 * args.layers)
    cp_us, cp_bytes = ctx.time_kernel(2, 20)
    log(f"gate|up {gu_us:.2f}us ({gu_bytes / gu_us / 1e3:.0f} GB/s), attention {at_us:.2f}us "
        f"({at_bytes / at_us / 1e3:.0f} GB/s), float4 copy 256 MiB {cp_bytes / cp_us / 1e3:.0f} GB/s")
    # the frame's fused launches standalone, as the frame runs them (direct
    # launches, HIP events): one talker layer at the current KV (3 launches)
    # and one predictor layer step (2 launches); per-launch durations and
    # counter bytes from the committed profile of bench.py --fused-only
    tl_us, tl_bytes = ctx.time_kernel(8, 4 * args.layers)
    pl_us, pl_bytes = ctx.time_kernel(9, 280)
    log(f"talker layer {tl_us:.2f}us ({tl_bytes / tl_us / 1e3:.0f} GB/s), predictor layer step {pl_us:.2f}us "
        f"({pl_bytes / pl_us / 1e3:.0f} GB/s)")
    prof = fused_profile()
    pmlp = next((v for k, v in prof.items() if k.startswith("predictor gate|up")), None)
    frame_kernels = {
        "talker_layer": {"launches": 3, "kv": ctx.kv_len() + 1, "us": round(tl_us, 2), "bytes": int(tl_bytes),
                         "gbs": round(tl_bytes / tl_us / 1e3, 1), "frac": round(tl_bytes / tl_us / 1e3 / HBM_PEAK_GBS, 4)},
        "predictor_layer_step": {"launches": 2, "us": round(pl_us, 2), "bytes": int(pl_bytes),
                                 "gbs": round(pl_bytes / pl_us / 1e3, 1),
                                 "frac": round(pl_bytes / pl_us / 1e3 / HBM_PEAK_GBS, 4)},
        "per_launch": prof, "source": os.path.relpath(FUSED_FILE, ROOT) if prof else None,
    }
    if pmlp:
        frame_kernels["roofline"] = {
            "bound": "hbm", "kernel": "k_mlp1<256, 4, 2, 1024, 1, 80> (predictor gate|up + down, one launch, one-group gate|up tiles)",
            "achieved": pmlp["alg_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": pmlp["frac"],
            "traffic": pmlp["counter_bytes"], "avg_us": pmlp["avg_us"], "bytes_per_launch": pmlp["alg_bytes"],
            "note": "from the committed kernel trace and counter passes (bench.py --fused-only)"}

    # Q4 GEMV k=2048 -> n=6144 (the GEMV tiles run inside every launch of
    # the frame) over a pool of distinct weights (> 256 MB
    # last-level cache); a streaming read of the same bytes in one launch
    # (its attainable bound); then the same kernel streaming a 113 MB weight
    grng = np.random.Generator(np.random.PCG64(1))
    pool = [ctx.upload(synth.q4_random(grng, 2048, 6144)) for _ in range(args.gemv_copies)]
    g_us, g_bytes = ctx.time_gemv(pool, 4 * args.gemv_copies)
    for w in pool:
        w.free()
    g_gbs = g_bytes / (g_us * 1e-6) / 1e9
    log(f"Q4 GEMV 2048x6144: {g_us:.2f}us/launch, {g_gbs:.0f} GB/s")
    r_us, r_bytes = ctx.time_kernel(7, 256)
    log(f"streaming read of the same {int(r_bytes)} B: {r_us:.2f}us/launch ({r_bytes / r_us / 1e3:.0f} GB/s)")
    traffic, traffic_src = measured_traffic(GEMV_KERNEL)
    roof = {"bound": "hbm", "achieved": round(g_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(g_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
            "kernel": f"{GEMV_KERNEL} (Q4 GEMV k=2048 -> n=6144, tile 1 group x 2048 rows)",
            "avg_us": round(g_us, 3), "bytes_per_launch": int(g_bytes), "traffic_source": traffic_src,
            "attainable": {"what": "streaming read of the same bytes in one launch (64 rotating 7.1 MB buffers)",
                           "us": round(r_us, 3), "gbs": round(r_bytes / r_us / 1e3, 1),
                           "gemv_over_read": round(g_us / r_us, 3)}}
    kernels = {
        "talker_gate_up_rmsnorm": {"us": round(gu_us, 2), "gbs": round(gu_bytes / gu_us / 1e3, 1),
                                   "bytes": int(gu_bytes)},
        f"talker_attention_kv{ctx.kv_len()}": {"us": round(at_us, 2), "gbs": round(at_bytes / at_us / 1e3, 1),
                                               "bytes": int(at_bytes)},
        "float4_copy_256MiB": {"us": round(cp_us, 2), "gbs": round(cp_bytes / cp_us / 1e3, 1),
                               "bytes": int(cp_bytes)},
    }
    if not args.no_stream:
        # the same kernel streaming one 113 MB weight per launch (4 copies);
        # --no-stream leaves it out, so that a profile's line for the kernel
        # covers the 2048 x 6144 launches alone
        big = synth.q4_random(grng, 2048, 98304)
        pool = [ctx.upload(big) for _ in range(4)]
        s_us, s_bytes = ctx.time_gemv(pool, 32)
        for w in pool:
            w.free()
        del big
        s_gbs = s_bytes / (s_us * 1e-6) / 1e9
        log(f"Q4 GEMV 2048x98304: {s_us:.2f}us/launch, {s_gbs:.0f} GB/s")
        kernels["q4_gemv_stream_2048x98304"] = {"us": round(s_us, 2), "gbs": round(s_gbs, 1),
                                                "frac": round(s_gbs / HBM_PEAK_GBS, 4), "bytes": int(s_bytes)}

    lg, hd, _, _ = ctx.gen_state()
    kernels["icl_prefill"] = time_prefill(ctx, args.layers)   # rewrites the KV cache
    if args.layers == 28 and not args.no_icl:
        kernels["icl_decode"] = time_icl_decode(ctx, params, pad)
    if not args.no_sweep:
        kernels["q4_gemv_shapes"] = gemv_sweep(ctx, synth)
        log("GEMV sweep: " + ", ".join(f"{k} {v['gbs']:.0f} GB/s" for k, v in kernels["q4_gemv_shapes"].items()))

    if not args.no_decoder:
        kernels["speech_decoder"] = time_decoder(synth, qtts, 0 if args.no_cpu else 120)

    cpu = None
    if not args.no_cpu:
        log("timing the CPU baseline (oracle)")
        cpu = cpu_baseline(talker, pred, lg, hd, pad, KV_HEADLINE, args.cpu_seconds)
        if cpu["isa"] != "avx2":
            a2 = cpu_baseline(talker, pred, lg, hd, pad, KV_HEADLINE, args.cpu_seconds / 2, isa="avx2")
            cpu["avx2"] = {"value": a2["value"], "sample": a2["sample"]}
        cpu["gemv_2048x6144"] = cpu_gemv()
        cpu["host"] = host_info()
        log(f"cpu baseline {cpu['value']:.3f} frames/s on {cpu['cores']} threads; GEMV {cpu['gemv_2048x6144']}")

    avg_bytes = float(np.mean([frame_bytes(kv_start + i) for i in range(frames)])) if args.layers == 28 else None
    frame_roof = None if avg_bytes is None else {
        "bound": "hbm", "bytes_per_frame_avg": int(avg_bytes), "bytes_per_frame_kv2048": frame_bytes(2048),
        "achieved": round(fps * avg_bytes / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(fps * avg_bytes / 1e9 / HBM_PEAK_GBS, 4),
        "note": "algorithmic bytes per frame (weights once + KV read and append) x frames/s"}
    out = {
        "metric": "codec frames/s (talker+predictor, batch 1) @KV 2048; Q4 GEMV HBM GB/s (% peak)",
        "value": round(fps, 3),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": frames,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * dt / max(frames, 1), 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random Q4 weights of the 1.7B shapes; random prompt ids)",
        "config": {"workload": f"frame loop at KV {kv_start}: {args.layers}-layer talker + 5-layer predictor, "
                               f"64-token prompt, frames from KV 64 untimed to {kv_start}, then {frames} timed "
                               f"frames KV {kv_start}->{kv_start + frames}, top-k 50, T 0.9, seed 42",
                   "kv_start": kv_start, "kv_end": kv_start + frames, "parallelism": "single GPU"},
        "frame_loop_from_prompt": loop,
        "roofline": roof,
        "frame_roofline": frame_roof,
        "device_memory_mb": mem,
        "frame_split": split,
        "frame_kernels": frame_kernels,
        "kernels": kernels,
        "cpu_baseline": cpu,
    }
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
