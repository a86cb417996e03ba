#!/usr/bin/env python3
"""Benchmark: qwen3-tts per-frame token loop on one MI355X.

Workload: the full frame loop at the reference 0.6B shapes with Q8_0 weights
(talker step + 2-token code-predictor prefill + 14 code-predictor steps per
frame, on-device sampling, one hipGraph launch per frame), batch 1, greedy,
after a 64-token synthetic prompt.  A "step" is one frame.  Weights are
seeded N(0, 0.02) (norm gains 1 + N(0, 0.02)), quantised with the converter's
Q8_0 formula.  EOS is biased off (eos_bias = -1e4, an argument of the
reference's generate()) so every timed frame does the full work.

Prints one JSON line: frames/s, ms per frame, the HBM roofline of the
dominant kernel and of the whole frame, and the CPU oracle's frames/s on the
same workload on this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qwen3-tts.cpp_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0


def frame_bytes(cfg, w, n_kv, cp_table=False):
    """Algorithmic HBM bytes of one frame: every weight byte once per pass
    that reads it (talker once; code predictor 15 passes; heads once per
    pass), plus KV reads/writes.  Activations are excluded (<0.1%).  n_kv is
    the talker KV length, or a list of lengths (one per stream) for the
    multi-stream loop, which reads every weight once per frame for all
    streams together.  cp_table: steps 1..14 take code-predictor layer 0's
    QKV rows from the per-code table (one fp32 row each) instead of reading
    that layer's QKV weights."""
    def nbytes(name):
        return w[name][2].nbytes
    talker = sum(nbytes(n) for n in w if n.startswith("talker.blk."))
    talker += nbytes("talker.codec_head.weight") + nbytes("talker.output_norm.weight")
    cp_layers = sum(nbytes(n) for n in w if n.startswith("code_pred.blk."))
    cp = 15 * (cp_layers + nbytes("code_pred.output_norm.weight")) + sum(
        nbytes(f"code_pred.lm_head.{g}.weight") for g in range(15))
    if "code_pred.mtp_proj.weight" in w:      # the 1.7B layout: each pass projects its input rows
        cp += 15 * (nbytes("code_pred.mtp_proj.weight") + nbytes("code_pred.mtp_proj.bias"))
    if cp_table:
        qkv0 = sum(nbytes(f"code_pred.blk.0.attn_{x}.weight") for x in "qkv") + nbytes("code_pred.blk.0.attn_norm.weight")
        qkvd = (cfg.n_head + 2 * cfg.n_kv_head) * cfg.head_dim
        cp -= 14 * qkv0
        cp += 14 * qkvd * 4
    kv_row = cfg.n_kv_head * cfg.head_dim * 2 * 2          # K and V, fp16
    per_stream = 0
    for n in (n_kv if isinstance(n_kv, (list, tuple)) else [n_kv]):
        talker_kv = cfg.n_layers * kv_row * (n + 1)          # read n rows + write 1
        cp_kv = cfg.cp_layers * kv_row * sum(g + 2 for g in range(15))
        embd = 17 * cfg.hidden_size * 2
        per_stream += talker_kv + cp_kv + embd
    return talker + cp + per_stream


def host_cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown cpu"


def cpu_baseline(cfg, w, text, spk, threads, budget_s):
    """Oracle (C++ CPU restatement) frames/s on the same workload: time two
    generate() calls of different length and difference them, so prefill
    and prompt projection cancel."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import q3t_oracle as orc
    o = orc.Oracle(cfg, w, threads=threads)
    global ORACLE_ISA
    ORACLE_ISA = os.path.basename(orc.LIB_PATH)
    t0 = time.perf_counter()
    o.generate(text, spk, max_len=1, temperature=0.0, eos_bias=-1e4)
    t1 = time.perf_counter()
    base = t1 - t0
    n2 = 3
    t0 = time.perf_counter()
    o.generate(text, spk, max_len=n2, temperature=0.0, eos_bias=-1e4)
    per = max((time.perf_counter() - t0 - base) / (n2 - 1), 1e-6)
    n3 = int(max(4, min(320, budget_s / per)))
    t0 = time.perf_counter()
    o.generate(text, spk, max_len=n3, temperature=0.0, eos_bias=-1e4)
    dt = time.perf_counter() - t0 - base
    o.close()
    return (n3 - 1) / dt, n3


# The CPU leg is the oracle: a scalar C++ restatement that accumulates every
# dot product in fp64.  ggml's x86 Q8_0 / F16 kernels (AVX2 / AVX-512 int8
# and fp32 SIMD) are not in this tree, so this figure very likely understates
# the reference's own CPU speed.
PORT_NOTE = ("CPU leg = the oracle (scalar C++ restatement, fp64 accumulation), not ggml's SIMD kernels: "
             "likely slower than the reference's CPU path")


def config1_leg(args, cfg, Device, driver, Weights):
    """Configuration 1 (F16 0.6B, 32-token prompt, greedy, 64 frames): the
    device frame loop timed with HIP events, and the oracle on 4 host threads
    over a bounded sample of the same workload."""
    w16 = Weights(cfg, "f16", seed=2024)
    rng = np.random.default_rng(18)
    text = rng.integers(0, cfg.text_vocab, 32).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)
    dev = Device(cfg, 0)
    dev.upload_weights(w16)
    pre, trail, pad = driver.build_prefill(dev, cfg, text, spk)
    plen = pre.shape[0]
    dev.kv_reserve(plen + 64 + 8)
    dev.prefill(pre, 0, want_hidden=False)
    dev.frames_begin(trail, pad, plen, 64, repetition_penalty=1.05, temperature=0.0, top_k=0, eos_bias=-1e4)
    dev.frames_run(8)
    us0, n0, _ = dev.frames_stats()
    codes, eos = dev.frames_run(56)
    us1, n1, path = dev.frames_stats()
    dev.close()
    assert not eos and codes.shape[0] == 56
    gpu_fps = (n1 - n0) / ((us1 - us0) * 1e-6)
    out = {"workload": "configuration 1: F16 0.6B shapes, 32-token prompt, greedy, 64 frames",
           "gpu_frames_per_s": round(gpu_fps, 2), "gpu_path": path,
           "gpu_sample": "frames 8..63 (HIP events around the frame launches)", "cpu": None}
    if not args.no_cpu_baseline:
        fps, n = cpu_baseline(cfg, w16, text, spk, 4, args.cpu_budget / 2)
        out["cpu"] = {"value": round(fps, 3), "unit": "frames/s", "cores": 4, "kind": "port",
                      "sample": f"oracle generate() of {n} frames minus a 1-frame run, 4 threads; {PORT_NOTE}"}
    return out


def prefill_bench(args, cfg, w):
    """One talker prefill of args.prefill rows (seeded N(0, 0.05) rows), the
    long-prompt half of the long-context configuration.  Q8_0 models take the
    int8 MFMA GEMM path; reports rows/s and the MFMA (int8) utilisation of the
    five GEMMs per layer against the 5.0 POP/s dense peak."""
    from qwen3_tts_amd.device import Device
    n = args.prefill
    dev = Device(cfg, 0)
    dev.upload_weights(w)
    dev.kv_reserve(n + 8)
    rows = (np.random.default_rng(21).standard_normal((n, cfg.hidden_size)) * 0.05).astype(np.float32)
    steps = max(args.steps, 1)

    def timed():
        for _ in range(max(args.warmup, 1)):
            dev.prefill(rows, 0, want_hidden=False)
        dev.sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            dev.prefill(rows, 0, want_hidden=False)
        return (time.perf_counter() - t0) / steps

    dt = timed()
    exact_ms = None
    if args.weights == "f16":
        # the exact f64-MFMA form of the F16 GEMMs beside the default fp16-MFMA one
        prev = os.environ.get("Q3T_PF_EXACT")
        os.environ["Q3T_PF_EXACT"] = "1"
        try:
            exact_ms = round(timed() * 1e3, 3)
        finally:
            if prev is None:
                del os.environ["Q3T_PF_EXACT"]
            else:
                os.environ["Q3T_PF_EXACT"] = prev
    dev.close()
    d, qd = cfg.hidden_size, cfg.n_head * cfg.head_dim
    qkvd = qd + 2 * cfg.n_kv_head * cfg.head_dim
    gemm_ops = 2.0 * n * cfg.n_layers * (qkvd * d + d * qd + 2 * cfg.ffn_size * d + d * cfg.ffn_size)
    fast = args.weights == "f16" and os.environ.get("Q3T_PF_EXACT", "0") != "1"
    print(json.dumps({
        "metric": "talker prefill rows/s (long prompt)", "value": round(n / dt, 1), "unit": "rows/s", "n_gpus": 1,
        "steps": steps, "warmup": max(args.warmup, 1), "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True,
        "dtype": "int8" if args.weights == "q8_0" else "f16", "data": "synthetic",
        "config": {"workload": f"talker prefill, {n} rows, {args.weights.upper()} 0.6B shapes", "rows": n,
                   "gemm": "int8 MFMA, fp64 block epilogue" if args.weights == "q8_0" else
                   ("fp16 MFMA, fp32 accumulation" if fast else "exact f64 MFMA")},
        "gemm_tops": round(gemm_ops / dt / 1e12, 2),
        "mfma_util": round(gemm_ops / dt / (5.0e15 if args.weights == "q8_0" else 2.5e15), 4),
        "exact_f64_form_ms": exact_ms}))


def step_bench(args, cfg, w):
    """One talker decode step (forward_step: 28 layers + output norm + codec
    head, batch 1) with the KV cache pre-filled at 512 positions with seeded
    N(0, 1) bfloat16-valued K/V rows, the new token at position 512.  Each
    call is one q3t_dev_talker_step (logits and hidden copied back to the
    host): the persistent kernel's talker pass for an fp16 cache, the
    multi-kernel step for a bfloat16 cache (--kv bf16).  Reports the mean wall
    time per step and the HIP event timings of the multi-kernel step's kernels
    for talker layer 0 at that context."""
    from qwen3_tts_amd.device import Device
    rng = np.random.default_rng(31)
    n_kv = 512
    dev = Device(cfg, 0)
    dev.upload_weights(w)
    if args.kv == "bf16":
        dev.kv_set_type(30)
    dev.kv_reserve(n_kv + 8)

    def bf16_bits(x):
        u = x.view(np.uint32)
        return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)

    for layer in range(cfg.n_layers):
        kv = [bf16_bits(rng.standard_normal((n_kv, cfg.n_kv_head, cfg.head_dim), dtype=np.float32)) for _ in range(2)]
        if args.kv == "f16":    # the same bfloat16 values, held exactly in fp16
            kv = [(b.astype(np.uint32) << np.uint32(16)).view(np.float32).astype(np.float16) for b in kv]
        dev.kv_write(layer, kv[0], kv[1])
    x = (rng.standard_normal(cfg.hidden_size) * 0.05).astype(np.float32)
    for _ in range(max(args.warmup, 1)):
        dev.talker_step(x, n_kv)
    steps = max(args.steps, 1)
    t0 = time.perf_counter()
    for _ in range(steps):
        dev.talker_step(x, n_kv)
    dt = (time.perf_counter() - t0) / steps
    step_path = {0: "multi-kernel step", 1: "persistent-kernel step (row-parallel program)",
                 3: "persistent-kernel step (XCD-parallel program)"}.get(dev.frames_stats()[2], "?")
    kernels = {}
    names = {0: "gemv_gate_up_swiglu", 1: "gemv_qkv_rmsnorm", 2: "gemv_down_resid", 3: "gemv_wo_resid",
             4: "attention_decode"}
    for k_, nm in names.items():
        us, b = dev.time_kernel(k_, 100)
        kernels[nm] = {"avg_us": round(us, 3), "bytes": int(b), "gbs": round(b / us / 1e3, 1) if us > 0 else None}
    dev.close()
    wbytes = sum(a.nbytes for n_, (_, _, a) in w.tensors.items() if n_.startswith("talker.blk.")) + \
        w.tensors["talker.codec_head.weight"][2].nbytes
    kvbytes = cfg.n_layers * cfg.n_kv_head * cfg.head_dim * 2 * 2 * (n_kv + 1)
    print(json.dumps({
        "metric": "talker decode step latency (KV 512)", "value": round(dt * 1e3, 4), "unit": "ms",
        "n_gpus": 1, "steps": steps, "warmup": max(args.warmup, 1), "ms_per_step": round(dt * 1e3, 4),
        "higher_is_better": False, "dtype": "int8" if args.weights == "q8_0" else "f16",
        "data": f"synthetic (seeded weights, N(0,1) bfloat16-valued K/V in a {args.kv} cache)",
        "config": {"workload": f"one talker decode step, {args.weights.upper()} 0.6B shapes, {args.kv} KV pre-filled to "
                               f"{n_kv} positions, {step_path} with host copy-back",
                   "global_batch": 1, "kv_type": args.kv},
        "step_algorithmic_bytes": int(wbytes + kvbytes),
        "step_hbm_gbs": round((wbytes + kvbytes) / dt / 1e9, 1),
        "kernels": kernels}))


def long_bench(args, cfg, w):
    """Long-context sampled decode: prefill rows [N(0,1) speaker row;
    text_proj(2048 uniform ids)] through one prefill call, then args.steps
    sampled frames (temperature 0.9, top-k 50, repetition penalty 1.05, fixed
    seed; EOS biased off so every frame does full work) while the talker
    context grows from 2049 to 2049 + warmup + steps positions.  Reports the
    prefill time and the decode frames/s with the HBM rate of the frame's
    algorithmic bytes at the mid-run context."""
    from qwen3_tts_amd.device import Device
    rng = np.random.default_rng(44)
    dev = Device(cfg, 0)
    dev.upload_weights(w)
    ids = rng.integers(0, cfg.text_vocab, args.long_prompt).astype(np.int32)
    spk = rng.standard_normal((1, cfg.hidden_size)).astype(np.float32)
    dev.text_proj(ids[:16])   # first-call set-up outside the timing
    # text projection of the prompt ids: tiled GEMMs (the product path for
    # 16 or more ids), and for comparison the 4-row GEMV chunks it replaced
    t0 = time.perf_counter()
    proj = dev.text_proj(ids)
    text_proj_s = time.perf_counter() - t0
    os.environ["Q3T_PREFILL_MFMA"] = "0"
    try:
        t0 = time.perf_counter()
        proj_gemv = dev.text_proj(ids)
        text_proj_gemv_s = time.perf_counter() - t0
    finally:
        del os.environ["Q3T_PREFILL_MFMA"]
    assert np.array_equal(proj, proj_gemv), "text projection: tiled and GEMV rows differ"
    rows = np.concatenate([spk, proj]).astype(np.float32)
    pad = dev.text_proj([cfg.tts_pad_id])[0]
    plen = rows.shape[0]
    total = args.warmup + args.steps
    dev.kv_reserve(plen + total + 8)
    # first-call set-up outside the timing: the prefill buffers grow to this row count once
    dev.prefill(rows, 0, want_hidden=False)
    t0 = time.perf_counter()
    dev.prefill(rows, 0, want_hidden=False)
    prefill_s = time.perf_counter() - t0
    dev.frames_begin(pad[None], pad, plen, total, repetition_penalty=1.05, temperature=args.temperature,
                     top_k=50 if args.temperature > 0 else 0, eos_bias=-1e4, seed=1234)
    if args.warmup:
        _, eos = dev.frames_run(args.warmup)
        assert not eos
    dev.sync()
    t0 = time.perf_counter()
    codes, eos = dev.frames_run(args.steps)
    elapsed = time.perf_counter() - t0
    us, n, path = dev.frames_stats()
    dev.close()
    assert not eos and codes.shape[0] == args.steps
    fps = args.steps / elapsed
    fbytes = frame_bytes(cfg, w.tensors, plen + args.warmup + args.steps // 2)
    print(json.dumps({
        "metric": "codec frames/sec, long-context sampled decode", "value": round(fps, 2), "unit": "frames/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(elapsed * 1e3 / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8" if args.weights == "q8_0" else "f16", "data": "synthetic (seeded weights, uniform ids)",
        "config": {"workload": f"{args.weights.upper()} 0.6B shapes, {plen}-row prefill (speaker row + text_proj of "
                               f"{args.long_prompt} ids), " + (f"sampled T={args.temperature} top-k 50" if
                               args.temperature > 0 else "greedy") + f", rep 1.05, context {plen} -> "
                               f"{plen + total}", "global_batch": 1, "prefill_rows": plen,
                   "frame_path": {0: "captured multi-kernel graph", 1: "persistent frame kernel"}.get(path, path)},
        "prefill_ms": round(prefill_s * 1e3, 2),
        "text_proj_ms": round(text_proj_s * 1e3, 2),
        "text_proj_gemv_chunks_ms": round(text_proj_gemv_s * 1e3, 2),
        "frame_algorithmic_bytes_mid": fbytes,
        "frame_hbm_gbs": round(fbytes * fps / 1e9, 1),
        "frame_roofline_frac": round(fbytes * fps / 1e9 / HBM_PEAK_GBS, 4)}))


def streams_bench(args, cfg, w):
    """Multi-stream batched decode: args.streams independent utterances, each
    a 128-token prompt (build_prefill rows) behind a seeded synthetic history
    so that its talker KV starts at a length drawn uniformly from
    [128, 2048]; greedy, EOS biased off, every stream advancing one frame per
    graph launch.  Reports aggregate frames/s over all streams, the int8 MFMA
    utilisation of the batched layer GEMMs against the 5.0 POP/s dense peak,
    and the HBM rate of the frame's algorithmic bytes (weights once per
    frame, every stream's KV)."""
    from qwen3_tts_amd import driver
    from qwen3_tts_amd.device import Device
    B = args.streams
    rng = np.random.default_rng(77)
    kv_len = rng.integers(128, 2049, B)
    dev = Device(cfg, 0)
    dev.upload_weights(w)
    total = args.warmup + args.steps
    n_ctx = int(kv_len.max()) + total + 8
    rows, plens = [], []
    for b in range(B):
        text = rng.integers(0, cfg.text_vocab, 128).astype(np.int32)
        spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)
        pre, trail, pad = driver.build_prefill(dev, cfg, text, spk)
        hist = (rng.standard_normal((int(kv_len[b]) - pre.shape[0], cfg.hidden_size)) * 0.05).astype(np.float32)
        rows.append((np.concatenate([hist, pre]).astype(np.float32), trail, pad))
    dev.streams_reserve(B, n_ctx)
    args_list = []
    for b, (ctx, trail, pad) in enumerate(rows):
        dev.stream_prefill(b, ctx)
        plens.append(ctx.shape[0])
        args_list.append(dict(trailing=trail, tts_pad=pad, n_past=ctx.shape[0], max_len=total, repetition_penalty=1.05,
                              temperature=0.0, top_k=0, eos_bias=-1e4))
    dev.streams_begin(args_list)
    if args.warmup:
        codes, eos = dev.streams_run(args.warmup)
        assert not any(eos)
    dev.sync()
    us0, n0, _ = dev.frames_stats()
    t0 = time.perf_counter()
    codes, eos = dev.streams_run(args.steps)
    elapsed = time.perf_counter() - t0
    us1, n1, path = dev.frames_stats()
    dev.close()
    assert path == 2 and not any(eos) and all(c.shape[0] == args.steps for c in codes), "stream stopped early"
    gpu_frame_s = (us1 - us0) * 1e-6 / max(n1 - n0, 1)
    fps = B * args.steps / elapsed
    d, qd = cfg.hidden_size, cfg.n_head * cfg.head_dim
    qkvd = qd + 2 * cfg.n_kv_head * cfg.head_dim
    layer_macs = qkvd * d + d * qd + 2 * cfg.ffn_size * d + d * cfg.ffn_size
    # talker: 1 row per stream per frame; code predictor: 2 + 14 rows per stream per frame
    frame_ops = 2.0 * B * layer_macs * (cfg.n_layers + 16 * cfg.cp_layers)
    fbytes = frame_bytes(cfg, w.tensors, [p + args.warmup + args.steps // 2 for p in plens])
    q8 = args.weights == "q8_0"
    # F16 layers: the fp16-MFMA GEMMs unless Q3T_MS_EXACT=1 selects the exact f64-MFMA ones
    f16_exact = os.environ.get("Q3T_MS_EXACT", "") == "1"
    # dense peaks: int8 MFMA 5.0 POP/s (Q8_0 layers), fp16 MFMA 2.5 PFLOP/s or f64 MFMA 78.6 TFLOP/s (F16 layers)
    peak = 5.0e15 if q8 else (78.6e12 if f16_exact else 2.5e15)
    out = {
        "metric": f"aggregate codec frames/sec, multi-stream batched decode {args.weights.upper()}", "value": round(fps, 1),
        "unit": "frames/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if q8 else ("f64 (fp16 operands)" if f16_exact else "fp16 (fp32 accumulation)"),
        "data": "synthetic (seeded weights, uniform prompt ids, N(0,0.05) history)",
        "config": {"workload": f"{B} streams, 128-token prompts, talker KV lengths uniform in [128, 2048], greedy, "
                               f"{args.weights.upper()} 0.6B shapes, one hipGraph per frame of all streams",
                   "global_batch": B, "frames_per_stream": args.steps, "kv_lengths": [int(x) for x in plens]},
        "gpu_ms_per_frame": round(gpu_frame_s * 1e3, 4),
        "per_stream_fps": round(args.steps / elapsed, 2),
        "layer_gemm_tops": round(frame_ops / gpu_frame_s / 1e12, 2),
        "mfma_util": round(frame_ops / gpu_frame_s / peak, 5),
        "frame_algorithmic_bytes": int(fbytes),
        "frame_hbm_gbs": round(fbytes / gpu_frame_s / 1e9, 1),
        "frame_roofline_frac": round(fbytes / gpu_frame_s / 1e9 / HBM_PEAK_GBS, 4),
    }
    print(json.dumps(out))


def voc_flops(c, n):
    """GEMM flops of one decode of an n-frame segment (the conv / linear
    products and the pre-transformer attention; element-wise work excluded)"""
    L, H, F = c.latent, c.hidden, c.ffn
    f = 2.0 * n * 3 * H * L + 2.0 * n * L * H + 2.0 * n * H * L
    f += c.n_layers * (2.0 * n * H * 3 * L + 2.0 * n * L * H + 2.0 * n * H * 2 * F + 2.0 * n * F * H
                       + 2.0 * (n * (n + 1) / 2) * L * 2)
    r = n
    for _ in range(2):
        f += 2.0 * r * L * L * 2
        r = (r - 1) * 2 + c.up_kernel
        f += 2.0 * r * L * c.cnx_ffn * 2
    ch = c.decoder_dim
    f += 2.0 * r * 7 * L * ch
    for s in c.rates:
        co = ch // 2
        f += 2.0 * s * (r - 1) * 2 * ch * co
        r = (r - 1) * s
        f += 3 * (2.0 * r * 7 * co * co + 2.0 * r * co * co)
        ch = co
    return f + 2.0 * r * 7 * ch


def vocoder_bench(args):
    """The streaming vocoder's unit of work: one decode_window of the
    reference's default stream shape (src/qwen3_tts.cpp:246-268: 48 frames of
    warm-up context + 25 new frames = 2 s of 24 kHz audio), at the 12 Hz
    tokenizer's decoder widths with seeded random weights.  Reports windows/s,
    the real-time factor (audio seconds per wall second) and the GEMM
    TFLOP/s against the 2.5 PFLOP/s dense fp16 MFMA peak."""
    from qwen3_tts_amd import vocoder as V
    c = V.full()
    w = V.VocWeights(c, seed=5)
    g = V.VocDevice(c, w)
    ctx, chunk = args.voc_context, args.voc_chunk
    n = ctx + chunk
    codes = np.random.default_rng(9).integers(0, c.codebook_size, (n, c.n_codebooks)).astype(np.int32)
    g.reserve(n)
    for _ in range(max(args.warmup, 1)):
        out = g.decode_window(codes, ctx, n, ctx)
    steps = max(args.steps, 1)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = g.decode_window(codes, ctx, n, ctx)
    dt = (time.perf_counter() - t0) / steps
    g.close()
    audio_s = out.size / 24000.0
    flops = voc_flops(c, n)
    cpu = None
    if not args.no_cpu_baseline:
        # the oracle on a bounded sample: a 2 + 2-frame window, scaled per new frame
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import q3t_oracle as orc
        o = orc.VocOracle(c, w, threads=args.cpu_threads_max)
        t0 = time.perf_counter()
        small = o.decode_window(codes[:4], 2, 4, 2)
        cdt = time.perf_counter() - t0
        o.close()
        cpu = {"value": round((small.size / 24000.0) / cdt, 4), "unit": "audio s per s", "cores": args.cpu_threads_max,
               "kind": "port", "sample": "oracle decode_window of 2 context + 2 new frames at full widths"}
    print(json.dumps({
        "metric": "vocoder decode_window real-time factor (audio s per s)", "value": round(audio_s / dt, 1),
        "unit": "audio s/s", "n_gpus": 1, "steps": steps, "warmup": max(args.warmup, 1),
        "ms_per_step": round(dt * 1e3, 3), "higher_is_better": True, "dtype": "f16 (fp32 accumulate)",
        "data": "synthetic", "config": {"workload": f"decode_window, {ctx} context + {chunk} new frames, 12 Hz "
                                                    f"tokenizer decoder widths", "frames": n,
                                        "samples_out": int(out.size)},
        "gemm_tflops": round(flops / dt / 1e12, 2), "mfma_frac_whole_window": round(flops / dt / 2.5e15, 4),
        "cpu_baseline": cpu}))


ORACLE_ISA = "liboracle.so"


def main():
    # the CPU-baseline leg loads the oracle build for the widest ISA level this
    # host supports (x86-64-v4 with AVX-512, else x86-64-v3)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    from q3t_oracle import host_isa
    if host_isa() == "v4" and os.path.exists(os.path.join(ROOT, "oracle", "liboracle_v4.so")):
        os.environ.setdefault("Q3T_ORACLE_ISA", "v4")
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--weights", default="q8_0", choices=["q8_0", "f16"])
    ap.add_argument("--prompt", type=int, default=64)
    ap.add_argument("--cpu-threads", type=int, default=4)
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--cpu-threads-max", type=int, default=16,
                    help="thread cap of the all-cores CPU baseline (the host share of one GPU)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-config1", dest="config1", action="store_false",
                    help="skip the configuration-1 leg (F16, 32-token prompt: device frames/s and the CPU oracle)")
    ap.add_argument("--kernel-iters", type=int, default=200,
                    help="launches per per-kernel timing of the multi-kernel path (0: skip)")
    ap.add_argument("--prefill", type=int, default=0,
                    help="instead of the frame loop, time one talker prefill of this many rows (Q8_0: int8 MFMA path)")
    ap.add_argument("--talker-step", action="store_true",
                    help="instead of the frame loop, time one talker decode step at a 512-position KV cache")
    ap.add_argument("--kv", default="f16", choices=["f16", "bf16"], help="--talker-step: talker KV cache type")
    ap.add_argument("--long", action="store_true",
                    help="instead of the short-prompt greedy loop, time long-context sampled decode after a long prefill")
    ap.add_argument("--long-prompt", type=int, default=2048, help="text ids of the --long prefill")
    ap.add_argument("--temperature", type=float, default=0.9, help="--long sampling temperature (0: greedy)")
    ap.add_argument("--model", default="0.6b", choices=["0.6b", "1.7b"],
                    help="frame-loop shapes: the 0.6B model (the headline) or the 1.7B layout (code_pred.mtp_proj)")
    ap.add_argument("--vocoder", action="store_true",
                    help="time the streaming vocoder's decode_window (48 context + 25 new frames)")
    ap.add_argument("--voc-context", type=int, default=48)
    ap.add_argument("--voc-chunk", type=int, default=25)
    ap.add_argument("--streams", type=int, default=0,
                    help="instead of batch 1, time multi-stream batched decode of this many streams (Q8_0)")
    ap.add_argument("--path", default="persistent", choices=["persistent", "graph"],
                    help="persistent: one cooperative kernel per frame; graph: the captured multi-kernel frame")
    args = ap.parse_args()
    os.environ["Q3T_FRAME_KERNEL"] = "1" if args.path == "persistent" else "0"
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (batch-1 decode is a single "
              "dependent chain; independent streams shard by data parallelism, one process per GPU).", file=sys.stderr)
        sys.exit(2)

    from qwen3_tts_amd import config, driver
    from qwen3_tts_amd.device import Device
    from qwen3_tts_amd.synth import Weights

    if args.vocoder:
        return vocoder_bench(args)
    cfg = config.full_17b() if args.model == "1.7b" else config.full_06b()
    w = Weights(cfg, args.weights, seed=2024)
    if args.prefill > 0:
        return prefill_bench(args, cfg, w)
    if args.streams > 0:
        return streams_bench(args, cfg, w)
    if args.long:
        return long_bench(args, cfg, w)
    if args.talker_step:
        return step_bench(args, cfg, w)
    rng = np.random.default_rng(12)
    text = rng.integers(0, cfg.text_vocab, args.prompt).astype(np.int32)
    spk = rng.standard_normal(cfg.hidden_size).astype(np.float32)

    dev = Device(cfg, 0)
    dev.upload_weights(w)
    driver.build_prefill(dev, cfg, text, spk)   # first-call set-up outside the timing
    t0 = time.perf_counter()
    pre, trail, pad = driver.build_prefill(dev, cfg, text, spk)
    build_s = time.perf_counter() - t0
    total = args.warmup + args.steps
    plen = pre.shape[0]
    dev.kv_reserve(plen + total + 8)
    dev.prefill(pre, 0, want_hidden=False)
    dev.frames_begin(trail, pad, plen, total, repetition_penalty=1.05, temperature=0.0, top_k=0, eos_bias=-1e4)
    if args.warmup:
        _, eos = dev.frames_run(args.warmup)
        assert not eos
    dev.sync()
    us0, n0, _ = dev.frames_stats()
    t0 = time.perf_counter()
    codes, eos = dev.frames_run(args.steps)
    elapsed = time.perf_counter() - t0
    us1, n1, path = dev.frames_stats()
    frame_kernel_us = (us1 - us0) / max(n1 - n0, 1)   # HIP events around the frame launches
    assert not eos and codes.shape[0] == args.steps, "EOS inside the timed region"
    ms_per_step = elapsed * 1000.0 / args.steps
    fps = args.steps / elapsed
    n_kv_mid = plen + args.warmup + args.steps // 2
    fbytes = frame_bytes(cfg, w.tensors, n_kv_mid, cp_table=path == 3 and os.environ.get("Q3T_CP_QKV_TABLE") != "0")

    # per-kernel HIP-event timing on the context's stream (talker layer 0)
    kernels = {}
    names = {0: "gemv_gate_up_swiglu", 1: "gemv_qkv_rmsnorm", 2: "gemv_down_resid", 3: "gemv_wo_resid",
             4: "attention_decode"}
    if args.kernel_iters > 0 or path not in (1, 3):
        for k, nm in names.items():
            us, b = dev.time_kernel(k, max(args.kernel_iters, 20))
            kernels[nm] = {"avg_us": round(us, 3), "bytes": int(b), "gbs": round(b / us / 1e3, 1) if us > 0 else None}
    # plain 64 MiB copy kernel: the achievable-bandwidth reference and the
    # calibration point for the FETCH_SIZE / WRITE_SIZE counters
    us, b = dev.time_kernel(5, 20)
    kernels["k_copy16 (64 MiB device copy)"] = {"avg_us": round(us, 3), "bytes": int(b), "gbs": round(b / us / 1e3, 1)}
    dev.close()
    traffic = None
    if path in (1, 3):
        # HBM-side bytes per k_frame dispatch from the FETCH_SIZE / WRITE_SIZE
        # counter runs (calibrated on a 64 MiB copy kernel), when committed
        tp = os.path.join(ROOT, "profiles", "k_frame_q8_0_06b_traffic.json")
        if args.weights == "q8_0" and args.model == "0.6b" and os.path.exists(tp):
            with open(tp) as f:
                traffic = json.load(f)["traffic_bytes_per_dispatch"]
        # the whole frame is one kernel: its roofline is the frame's algorithmic bytes over its duration
        dom_name = "k_frame (persistent cooperative frame kernel, 256 workgroups x 256 threads)"
        dom = {"avg_us": round(frame_kernel_us, 3), "bytes": fbytes, "gbs": round(fbytes / frame_kernel_us / 1e3, 1)}
        kernels["k_frame"] = dom
    else:
        dom_name = "gemv_gate_up_swiglu (talker layer 0, Q8_0 1024->2x3072)"
        dom = kernels["gemv_gate_up_swiglu"]

    cpu = cpu_all = None
    if not args.no_cpu_baseline:
        nthreads = args.cpu_threads
        host = f"{host_cpu_model()}, {os.cpu_count()} host cpus"
        cpu_fps, n_frames = cpu_baseline(cfg, w, text, spk, nthreads, args.cpu_budget)
        cpu = {"value": round(cpu_fps, 3), "unit": "frames/s", "cores": nthreads, "kind": "port",
               "sample": f"oracle generate() of {n_frames} frames minus a 1-frame run, same weights/prompt, "
                         f"{nthreads} threads; {host}; {ORACLE_ISA} (-march=x86-64-"
                         f"{'v4' if 'v4' in ORACLE_ISA else 'v3'}, the host's widest level). " + PORT_NOTE}
        # the same leg on all the host cores this process may use (capped at
        # the GPU's share of them), with half the time budget
        nall = min(len(os.sched_getaffinity(0)), args.cpu_threads_max)
        if nall > nthreads:
            fps_all, n_all = cpu_baseline(cfg, w, text, spk, nall, args.cpu_budget / 2)
            cpu_all = {"value": round(fps_all, 3), "unit": "frames/s", "cores": nall, "kind": "port",
                       "sample": f"as cpu_baseline with {nall} threads, {n_all} frames; {host}"}

    config1 = None
    if args.config1 and args.model == "0.6b":
        config1 = config1_leg(args, cfg, Device, driver, Weights)

    out = {
        "metric": "codec frames/sec at batch 1 Q8_0 (RTF vs 12 Hz); achieved HBM GB/s per step",
        "value": round(fps, 2),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if args.weights == "q8_0" else "f16",
        "data": "synthetic (seeded N(0,0.02) weights, uniform prompt ids)",
        "config": {"workload": f"full frame loop, {args.weights.upper()} {args.model.upper()} shapes, {args.prompt}-token prompt, "
                               f"greedy, " + ("one persistent kernel per frame" + (", XCD-parallel layers" if path == 3 else "") if path in (1, 3) else "hipGraph per frame"),
                   "global_batch": 1, "frames": args.steps,
                   "weights": args.weights, "prompt_tokens": args.prompt, "prefill_rows": plen},
        "prefill_build_ms": round(build_s * 1e3, 3),
        "rtf_12hz": round(fps / 12.0, 2),
        "rtf_12_5hz": round(fps / 12.5, 2),
        "frame_algorithmic_bytes": fbytes,
        "frame_hbm_gbs": round(fbytes / (ms_per_step * 1e-3) / 1e9, 1),
        "frame_roofline_frac": round(fbytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "roofline": {"bound": "hbm", "achieved": dom["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dom["gbs"] / HBM_PEAK_GBS, 4) if dom["gbs"] else None, "traffic": traffic,
                     "kernel": dom_name},
        "kernels": kernels,
        "cpu_baseline": cpu,
        "cpu_baseline_all_cores": cpu_all,
        "config1": config1,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
