#!/usr/bin/env python3
"""Decode throughput of the HIP path on one MI355X (BASELINE.json metric).

Workload: synthetic Llama-3-8B-shape Q4_K_M model
(32 layers, d_model 4096, 32 q / 8 kv heads, head_dim 128, SwiGLU 14336, vocab
128256, RoPE theta 500000; Q4_K attn_q/k/o + ffn_gate/up, Q6_K attn_v, half of
ffn_down and the output head), weights N(0, 0.02) from a seed, batch 1, KV
cache prefilled with random token ids to ctx 4096, then greedy decode with the
reference's repeat penalty 1.1.  A "step" is one decode token: embedding ->
32 layers -> logits -> on-device greedy pick, replayed as one HIP graph.

Also measured in the same run:
- roofline: the dominant kernel, exact decode attention of one layer (the
  streamed launch: scores, coefficients and recurrence in one grid; or the
  separate launches where a shape takes those): the K and V bytes it must
  read at the profiled positions over the launch's (launches') average
  duration, timed with HIP events on the library stream during a profiling
  pass of the same decode;
- roofline_gemv: the fused gate/up Q4_K GEMV (SwiGLU epilogue), the largest
  per-launch weight stream, timed the same way;
- cpu_baseline: the CPU oracle (C restatement of the reference's AVX2 path,
  oracle/) continuing the same decode from the GPU's KV cache on the host's
  cores, for a bounded sample of tokens;
- prefill: batched prefill of the first --prefill-tokens prompt tokens
  (forward_prefill_batch on the device), tok/s and the int8 MFMA roofline of
  its fused gate/up product.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s Llama-3-8B-shape Q4_K_M bs1 ctx4096; GEMV HBM GB/s vs peak"
HBM_PEAK_GBS = 8000.0


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, int(os.environ.get("OMP_NUM_THREADS", n))))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--config", default="llama3-8b-q4km")
    ap.add_argument("--ctx", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--penalty", type=float, default=1.1)
    ap.add_argument("--profile-tokens", type=int, default=8)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--kv-fill", choices=["prefill", "random"], default="prefill",
                    help="prefill: run the ctx random-id prompt through the decoder; random: write N(0,1) K/V "
                         "directly (same per-token decode work, far fewer dispatches, for profiler runs)")
    ap.add_argument("--prefill-tokens", type=int, default=512,
                    help="prompt length of the batched-prefill measurement (0: skip it)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="run only the batched-prefill measurement and print its JSON object")
    ap.add_argument("--sweep", action="store_true",
                    help="run only the isolated kernel sweep (BASELINE configs[1]): batch-1 GEMV per format and "
                         "shape, and GQA decode attention at ctx 512/4096/32768; prints one JSON object")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="run only a plain device copy (y = x * 1) over this many MiB, 5 launches, and exit: the "
                         "known-size kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return
    if args.sweep:
        kernel_sweep(args)
        return

    import numpy as np
    from rustyllm_amd import hip, synth

    if not hip.available():
        raise SystemExit("rusty_hip_available() == 0: no gfx950 device")
    if args.config in synth.GPTOSS_CONFIGS:
        bench_gptoss(args)
        return

    t0 = time.time()
    model = synth.make_model(args.config, seed=args.seed)
    cfg = model["config"]
    log(f"model {args.config} generated in {time.time() - t0:.1f}s, {synth.weight_bytes(model) / 1e9:.3f} GB weights")

    cpu_slots = 0 if args.no_cpu else 256
    storage = args.ctx + args.warmup + args.steps + args.profile_tokens + 8 + cpu_slots
    t0 = time.time()
    res = hip.Resident(model, storage_len=storage)
    log(f"uploaded to HBM in {time.time() - t0:.1f}s (storage {storage} slots)")

    prompt = synth.token_ids(args.seed + 1, args.ctx, cfg["vocab"]).astype(np.int32)
    prefill = None
    if args.prefill_tokens and (args.kv_fill == "prefill" or args.prefill_only):
        prefill = measure_prefill(hip, res, prompt[:min(args.prefill_tokens, args.ctx)], cfg, log)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill}), flush=True)
        return

    # KV prefill: ctx random-id positions (all but the last through batched
    # prefill), then `warmup` greedy tokens.
    t0 = time.time()
    if args.kv_fill == "prefill":
        res.generate(prompt, args.warmup, penalty=args.penalty, want_logits=False)
    else:
        w = cfg["n_kv_heads"] * cfg["head_dim"]
        for layer in range(cfg["n_layers"]):
            for which in (0, 1):
                res.kv_write(layer, which, 0, synth.normal_f32(args.seed + 7 * layer + which, args.ctx - 1, w, 1.0))
        res.generate(prompt[-1:], args.warmup, penalty=args.penalty, start_pos=args.ctx - 1, want_logits=False)
    log(f"KV fill ({args.kv_fill}) {args.ctx} + warmup {args.warmup} tokens in {time.time() - t0:.1f}s")

    # ---- timed region: `steps` decode tokens, HIP events on the library stream
    ms = res.time_decode(args.steps, penalty=args.penalty)
    tok_s = args.steps / (ms / 1e3)
    log(f"decode {args.steps} tokens: {ms:.2f} ms -> {tok_s:.1f} tok/s")

    # ---- profiling pass: per-launch events, graphs bypassed ---------------------
    hip.profile_enable(True)
    prof_ms = res.time_decode(args.profile_tokens, penalty=args.penalty)
    prof = hip.profile_results()
    hip.profile_enable(False)
    fam_tot = sorted(((k, v) for k, v in prof.items() if v[1] > 0), key=lambda kv: -kv[1][0])
    log("profile (per token): " + ", ".join(
        f"{k}={v[0] / args.profile_tokens:.3f}ms/{v[1] // args.profile_tokens}" for k, v in fam_tot))

    dim, hid = cfg["dim"], cfg["hidden_dim"]
    nb = dim // 256
    swiglu_bytes = 2 * hid * nb * 144 + 2 * dim * 4 + hid * 4  # gate+up blocks, x and the norm weights, y
    tot, cnt = prof.get("gemv_kquant_swiglu", (0.0, 0))
    avg_ms = tot / cnt if cnt else float("nan")
    achieved = swiglu_bytes / (avg_ms * 1e-3) / 1e9 if cnt else 0.0

    # whole-token algorithmic bytes: every weight once + attended KV
    kv_per_tok = cfg["n_layers"] * 2 * cfg["n_kv_heads"] * cfg["head_dim"] * 4
    pos_mid = args.ctx + args.warmup + args.steps // 2
    token_bytes = synth.weight_bytes(model) + kv_per_tok * pos_mid
    eff_gbs = token_bytes * tok_s / 1e9

    traffic = recorded_traffic(args)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(model, res, storage, args, log)

    # exact attention of one layer: K and V rows of every attended position
    # (the profiling pass decodes positions p0 .. p0 + profile_tokens - 1,
    # each attending p + 1 positions) plus q and the outputs
    roofline = None
    fams = ATTN_STREAM_FAMS if ATTN_STREAM_FAMS[0] in prof else ATTN_FAMS
    attn_parts = {f: prof[f][0] / prof[f][1] for f in fams if f in prof and prof[f][1]}
    if len(attn_parts) == len(fams):
        p0 = args.ctx - 1 + args.warmup + args.steps
        n_att = p0 + 1 + (args.profile_tokens - 1) / 2
        hd = cfg["head_dim"]
        attn_bytes = int(n_att * cfg["n_kv_heads"] * 2 * hd * 4 + cfg["n_heads"] * 2 * hd * 4)
        attn_ms = sum(attn_parts.values())
        attn_gbs = attn_bytes / (attn_ms * 1e-3) / 1e9
        roofline = {
            "kernel": "exact attention per layer: %s (%d q / %d kv heads, head_dim %d, %.1f positions)"
                      % (" + ".join(fams), cfg["n_heads"], cfg["n_kv_heads"], hd, n_att),
            "bound": "hbm",
            "achieved": round(attn_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(attn_gbs / HBM_PEAK_GBS, 4),
            "traffic": recorded_traffic(args, ATTN_TRAFFIC_FILE),
            "bytes_per_launch": attn_bytes,
            "avg_launch_us": round(attn_ms * 1e3, 3),
            "avg_launch_us_parts": {f: round(v * 1e3, 3) for f, v in attn_parts.items()},
            "launches": prof[fams[-1]][1],
        }
    roofline_gemv = None
    if cnt:
        roofline_gemv = {
            "kernel": "gemv_kquant_swiglu (Q4_K gate+up %dx%d x2, SwiGLU epilogue)" % (hid, dim),
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "bytes_per_launch": swiglu_bytes,
            "avg_launch_us": round(avg_ms * 1e3, 3),
            "launches": cnt,
        }
    metric = METRIC if args.config == "llama3-8b-q4km" and args.ctx == 4096 else \
        f"decode tok/s {args.config} bs1 ctx{args.ctx}"
    line = {
        "metric": metric,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xq8_0->f32" if cfg["quant"] == "q8_0" else "int8xq4k/q6k->f32",
        "data": "synthetic",
        "config": {
            "workload": f"{args.config} greedy decode bs1, KV prefilled to ctx {args.ctx}",
            "ctx": args.ctx, "layers": cfg["n_layers"], "d_model": dim, "heads": [cfg["n_heads"], cfg["n_kv_heads"]],
            "head_dim": cfg["head_dim"], "ffn": hid, "vocab": cfg["vocab"], "quant": cfg["quant"],
            "repeat_penalty": args.penalty, "seed": args.seed,
        },
        "roofline": roofline,
        "roofline_gemv": roofline_gemv,
        "token_bytes": token_bytes,
        "effective_GBps": round(eff_gbs, 1),
        "effective_frac": round(eff_gbs / HBM_PEAK_GBS, 4),
        "profile_ms_per_token": {k: round(v[0] / args.profile_tokens, 4) for k, v in fam_tot},
        "profile_pass_ms_per_token": round(prof_ms / args.profile_tokens, 4),
        "cpu_baseline": cpu,
        "prefill": prefill,
    }
    print(json.dumps(line), flush=True)


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 MFMA


def bench_gptoss(args):
    """BASELINE.json configs[4] (not the headline): the gpt-oss decode step
    on the resident decoder in MoE mode.  KV is filled with N(0,1) values to
    ctx (the reference prefills gpt-oss token by token; the fill only sets the
    attended context), then `steps` greedy tokens are timed as for the
    standard models.  Bytes per token: the Q8_0 attention and router weights,
    the top-k experts' MXFP4 rows, the output head, and the attended KV
    (128-position window on even layers, the whole context on odd ones)."""
    import numpy as np
    from rustyllm_amd import hip, synth

    t0 = time.time()
    model = synth.make_gptoss(args.config, seed=args.seed)
    cfg = model["config"]
    log(f"model {args.config} generated in {time.time() - t0:.1f}s")
    cpu_slots = 0 if args.no_cpu else 512
    storage = args.ctx + args.warmup + args.steps + args.profile_tokens + 8 + cpu_slots
    res = hip.ResidentGptOss(model, max(storage, args.prefill_tokens + 1))
    prefill = None
    if args.prefill_tokens:
        # BASELINE configs[4]'s prompt: batched prefill of prefill_tokens ids
        prompt_pf = synth.token_ids(args.seed + 2, args.prefill_tokens, cfg["vocab"]).astype(np.int32)
        prefill = measure_prefill_gptoss(hip, res, prompt_pf, log)
    if args.prefill_only:
        print(json.dumps({"prefill": prefill}), flush=True)
        return
    kd = cfg["n_kv_heads"] * cfg["head_dim"]
    # the cache is the reference's ring of min(window, max_len) slots: random
    # rows in every slot stand for the last positions before ctx - 1
    n_fill = min(args.ctx - 1, res.slots)
    for layer in range(cfg["n_layers"]):
        for which in (0, 1):
            res.kv_write(layer, which, 0, synth.normal_f32(args.seed + 7 * layer + which, n_fill, kd, 1.0))
    prompt = synth.token_ids(args.seed + 1, 4, cfg["vocab"]).astype(np.int32)
    res.generate(prompt[-1:], args.warmup, penalty=args.penalty, start_pos=args.ctx - 1, want_logits=False)
    ms = res.time_decode(args.steps, penalty=args.penalty)
    tok_s = args.steps / (ms / 1e3)
    log(f"decode {args.steps} tokens: {ms:.2f} ms -> {tok_s:.1f} tok/s")
    hip.profile_enable(True)
    res.time_decode(args.profile_tokens, penalty=args.penalty)
    prof = hip.profile_results()
    hip.profile_enable(False)
    fam = sorted(((k, v) for k, v in prof.items() if v[1] > 0), key=lambda kv: -kv[1][0])
    log("profile (per token): " + ", ".join(f"{k}={v[0] / args.profile_tokens:.3f}ms/{v[1] // args.profile_tokens}"
                                             for k, v in fam))
    dim, hid, k, ne = cfg["dim"], cfg["hidden_dim"], cfg["top_k"], cfg["n_experts"]
    L0 = model["layers"][0]
    per_layer = sum(L0[n][0].nbytes for n in ("wq", "wk", "wv", "wo")) + L0["router"].nbytes
    per_layer += k * (L0["gate_exps"].nbytes + L0["up_exps"].nbytes + L0["down_exps"].nbytes) // ne
    pos = args.ctx + args.warmup + args.steps // 2
    kv = sum(min(pos, cfg["window"]) if l % 2 == 0 else pos for l in range(cfg["n_layers"])) * 2 * kd * 4
    token_bytes = cfg["n_layers"] * per_layer + model["output"][0].nbytes + kv
    eff = token_bytes * tok_s / 1e9
    # dominant kernel family: the routed experts' MXFP4 products (per layer one
    # gate/up launch over the k experts' 2 x hidden rows and one down launch
    # over their dim rows); algorithmic bytes = the k experts' blocks + x + y
    roofline = None
    tot, cnt = prof.get("gemv_mxfp4", (0.0, 0))
    if cnt:
        exp_bytes = k * (L0["gate_exps"].nbytes + L0["up_exps"].nbytes + L0["down_exps"].nbytes) // ne
        act_bytes = k * (2 * (dim * 4 + hid * 4) + (hid * 4 + dim * 4))
        bytes_per_launch = (exp_bytes + act_bytes) / 2.0
        avg_ms = tot / cnt
        gbs = bytes_per_launch / (avg_ms * 1e-3) / 1e9
        roofline = {
            "kernel": "gemv_mxfp4 (top-%d of %d experts, gate+up %dx%d and down %dx%d MXFP4 rows, reference "
                      "serial row sums)" % (k, ne, 2 * hid, dim, dim, hid),
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None, "bytes_per_launch": int(bytes_per_launch),
            "avg_launch_us": round(avg_ms * 1e3, 3), "launches": cnt,
        }
    cpu = None if args.no_cpu else cpu_baseline_gptoss(model, res, args, log)
    line = {
        "metric": "decode tok/s gpt-oss-20B-shape MXFP4 MoE bs1 ctx%d" % args.ctx,
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32xmxfp4/q8_0->f32", "data": "synthetic",
        "config": {"workload": f"{args.config} greedy decode bs1, KV filled to ctx {args.ctx}", "ctx": args.ctx,
                   "layers": cfg["n_layers"], "d_model": dim, "experts": [ne, k], "window": cfg["window"],
                   "seed": args.seed},
        "roofline": roofline,
        "token_bytes": token_bytes,
        "effective_GBps": round(eff, 1),
        "effective_frac": round(eff / HBM_PEAK_GBS, 4),
        "profile_ms_per_token": {kk: round(v[0] / args.profile_tokens, 4) for kk, v in fam},
        "cpu_baseline": cpu,
        "prefill": prefill,
    }
    print(json.dumps(line), flush=True)


def cpu_baseline_gptoss(model, res, args, log):
    """The CPU oracle's gpt-oss decode step (orc_gptoss_forward: the C
    restatement of forward_gpt_oss_into with the reference's ring cache)
    continues from the GPU's ring KV at the same position, bounded sample.
    It runs on the reference's own schedule (orc_set_fast_schedule(0): MXFP4
    rows one dot_mxfp4_f32_scalar call each in the 64-row worker split, the
    sink loop's heads one after another), not the checker's faster one."""
    from oracle import oracle as O

    cfg = model["config"]
    cores = host_cores()
    t0 = time.time()
    pos0 = args.ctx + args.warmup + args.steps + args.profile_tokens - 1
    orc = O.OracleGptOss(model, res.storage_len, threads=cores)
    S = orc.storage
    for layer in range(cfg["n_layers"]):
        orc.kc[layer][:] = res.kv_read(layer, 0, 0, S)
        orc.vc[layer][:] = res.kv_read(layer, 1, 0, S)
    log(f"cpu baseline: ring KV copied in {time.time() - t0:.1f}s, {cores} threads")
    tok, n, pos = 1, 0, pos0
    t_start = time.time()
    O.lib.orc_set_fast_schedule(0)
    try:
        while pos < res.storage_len and (n < 2 or time.time() - t_start < args.cpu_seconds):
            logits = orc.forward(tok, pos)
            tok, _ = O.greedy(logits, [], 1.0)
            pos += 1
            n += 1
    finally:
        O.lib.orc_set_fast_schedule(1)
    dt = time.time() - t_start
    v = n / dt
    log(f"cpu baseline: {n} tokens in {dt:.1f}s -> {v:.2f} tok/s")
    return {"value": round(v, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode tokens of the same gpt-oss-20B-shape model at positions "
                      f"{pos0}..{pos0 + n} (C restatement of the reference x86 path, {cores} threads)"}


def measure_prefill_gptoss(hip, res, toks, log):
    """Batched gpt-oss prefill (rusty_hip_resident_prefill in MoE mode) of
    `toks` from position 0: whole-call wall time on the host clock around the
    synchronous call, then a profiling pass for per-launch times.  The
    reference prefills gpt-oss one decode step per token."""
    n = int(toks.size)
    if not res.prefill(toks, 0):  # warm-up (allocates the chunk buffers)
        log("prefill: model not batchable")
        return None
    t0 = time.perf_counter()
    res.prefill(toks, 0)
    sec = time.perf_counter() - t0
    hip.profile_enable(True)
    res.prefill(toks, 0)
    prof = hip.profile_results()
    hip.profile_enable(False)
    mfma = hip.set_expert_mfma(False)  # read the setting back
    hip.set_expert_mfma(mfma)
    log(f"prefill {n} tokens ({'matrix-core' if mfma else 'serial'} expert product): {sec * 1e3:.1f} ms -> "
        f"{n / sec:.1f} tok/s")
    fam = sorted(((k, v) for k, v in prof.items() if v[1] > 0), key=lambda kv: -kv[1][0])
    log("prefill profile: " + ", ".join(f"{k}={v[0]:.2f}ms/{v[1]}" for k, v in fam[:12]))
    # the expert gate/up products: 2 x (tokens x top_k pairs) x (2 x hidden
    # rows) x d_model f32 operations per layer, over all of the prefill's
    # launches (one per layer and chunk)
    cfg = res.cfg
    ops = 2.0 * n * cfg["top_k"] * 2 * cfg["hidden_dim"] * cfg["dim"] * cfg["n_layers"]
    tot, cnt = prof.get("pf_mxfp4_gate_up", (0.0, 0))
    tflops = ops / (tot * 1e-3) / 1e12 if cnt else 0.0
    roofline = {"kernel": "pf_mxfp4_gate_up (%s: %d pairs x %d rows x %d, f32)"
                % ("gemm_mxfp4_experts_mfma_kernel, f32 MFMA" if mfma else
                   "gemv_mxfp4_experts_kernel, serial reference-order sums", n * cfg["top_k"],
                   2 * cfg["hidden_dim"], cfg["dim"]),
                "bound": "mfma" if mfma else "valu", "achieved": round(tflops, 2), "peak": FP32_PEAK_TFLOPS,
                "unit": "TFLOP/s", "frac": round(tflops / FP32_PEAK_TFLOPS, 4),
                "ops_per_launch": ops / cnt if cnt else None,
                "avg_launch_us": round(tot / cnt * 1e3, 1) if cnt else None, "launches": cnt}
    return {"tokens": n, "tok_s": round(n / sec, 1), "ms": round(sec * 1e3, 2),
            "experts": "mfma" if mfma else "serial", "roofline": roofline,
            "profile_ms": {k: round(v[0], 3) for k, v in fam}}


def measure_prefill(hip, res, toks, cfg, log):
    """Batched prefill (rusty_hip_resident_prefill) of `toks` from position 0:
    whole-call wall time (host clock around the synchronous call; the tokens
    are uploaded inside it), then a profiling pass for per-launch times.  The
    MFMA roofline is the fused gate/up batched product: 2*ffn*d_model*T int8
    operations per launch, T = the chunk's tokens."""
    n = int(toks.size)
    res.prefill(toks, 0)  # warm-up (allocates the chunk buffers)
    t0 = time.perf_counter()
    ok = res.prefill(toks, 0)
    sec = time.perf_counter() - t0
    if not ok:
        log("prefill: model not batchable")
        return None
    hip.profile_enable(True)
    res.prefill(toks, 0)
    prof = hip.profile_results()
    hip.profile_enable(False)
    chunk = min(n, int(os.environ.get("RUSTY_HIP_PREFILL_CHUNK", "512")))
    tot, cnt = prof.get("pf_gemm_gate_up", (0.0, 0))
    avg_ms = tot / cnt if cnt else float("nan")
    ops = 2.0 * cfg["hidden_dim"] * cfg["dim"] * chunk
    tops = ops / (avg_ms * 1e-3) / 1e12 if cnt else 0.0
    log(f"prefill {n} tokens: {sec * 1e3:.1f} ms -> {n / sec:.1f} tok/s; gate/up product {avg_ms * 1e3:.1f} us "
        f"= {tops:.1f} TOP/s")
    return {
        "tokens": n,
        "tok_s": round(n / sec, 1),
        "ms": round(sec * 1e3, 2),
        "chunk": chunk,
        "roofline": {
            "kernel": "pf_gemm_gate_up (Q4_K %dx%d x %d tokens, i8 MFMA)" % (cfg["hidden_dim"], cfg["dim"], chunk),
            "bound": "mfma",
            "achieved": round(tops, 1),
            "peak": INT8_PEAK_TOPS,
            "unit": "TOP/s",
            "frac": round(tops / INT8_PEAK_TOPS, 4),
            "ops_per_launch": ops,
            "avg_launch_us": round(avg_ms * 1e3, 2),
            "launches": cnt,
        },
        "profile_ms": {k: round(v[0], 3) for k, v in sorted(prof.items(), key=lambda kv: -kv[1][0]) if v[1] > 0},
    }


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_kquant_swiglu_llama3-8b-q4km_traffic.json")
ATTN_TRAFFIC_FILE = os.path.join(ROOT, "profiles", "attention_exact_llama3-8b-q4km_ctx4096_traffic.json")
ATTN_FAMS = ("attn_exact_scores", "attn_exact_coef", "attn_exact_chain")
ATTN_STREAM_FAMS = ("attn_exact_stream",)


# (block elements, block bytes) per GGML type, and the kernel family that
# serves a batch-1 GEMV of that type at K % 256 == 0
SWEEP_FORMATS = {"q8_0": (8, 32, 34, "gemv_q8_0_int"), "q4_k": (12, 256, 144, "gemv_kquant"),
                 "q6_k": (14, 256, 210, "gemv_kquant"), "mxfp4": (39, 32, 17, "gemv_mxfp4")}
SWEEP_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336), (128256, 4096)]
SWEEP_CTX = [512, 4096, 32768]
COLD_BYTES = 640e6  # rotate inputs over more than the 256 MB memory-side cache + 32 MB of L2


def kernel_sweep(args):
    """Isolated kernel sweep.  Each GEMV streams
    W ~ N(0, 0.02) quantized by this repo's quantizers, x ~ N(0, 1); x is
    quantized to Q8_K on the device for Q8_0/Q4_K/Q6_K (all K here are
    multiples of 256) and stays f32 for MXFP4, as in the reference.  Weights
    and K/V rotate over enough device copies to exceed the caches.  Time per
    launch is the dispatch-stamped kernel duration (profile families)."""
    import numpy as np
    from rustyllm_amd import hip, synth

    if not hip.available():
        raise SystemExit("rusty_hip_available() == 0: no gfx950 device")
    gemv = []
    for name, (t, be, bb, fam) in SWEEP_FORMATS.items():
        for n, k in SWEEP_SHAPES:
            w = synth.normal_quantized(t, args.seed + n + k, n, k, 0.02)
            x = synth.normal_f32(args.seed + 1, 1, k, 1.0)[0]
            alg = n * (k // be) * bb + 4 * k + 4 * n
            copies = int(min(64, max(2, -(-COLD_BYTES // w.nbytes))))
            iters = max(24, 2 * copies) if w.nbytes < 100e6 else 12
            hip.bench_matvec(t, w, x, n, k, 2, 2)  # warm: upload, first launches
            hip.profile_enable(True)
            y = hip.bench_matvec(t, w, x, n, k, copies, iters)
            prof = hip.profile_results()
            hip.profile_enable(False)
            hip.weight_cache_clear()
            tot, cnt = prof.get(fam, (0.0, 0))
            if not cnt or not np.all(np.isfinite(y)):
                raise SystemExit(f"sweep {name} {n}x{k}: no {fam} launches recorded or non-finite output")
            us = tot / cnt * 1e3
            gbs = alg / (us * 1e-6) / 1e9
            gemv.append({"format": name, "rows": n, "cols": k, "kernel": fam, "alg_bytes": alg,
                         "avg_launch_us": round(us, 3), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "launches": cnt, "copies": copies})
            log(f"gemv {name:5s} {n:6d}x{k:5d}: {us:8.2f} us  {gbs:7.1f} GB/s  frac {gbs / HBM_PEAK_GBS:.3f}")
    attn = []
    heads, kv_mul, hd = 32, 4, 128
    n_kv = heads // kv_mul
    # exact: the coefficient launch runs only where the chain workgroups do not
    # compute the coefficients themselves
    fams = {"exact": ["attn_exact_scores", "attn_exact_coef", "attn_exact_chain", "attn_exact_finish"],
            "fast": ["attn_partial", "attn_combine"]}
    optional = {"attn_exact_coef"}
    for ctx in SWEEP_CTX:
        alg = ctx * n_kv * (hd + hd) * 4 + 4 * heads * (hd + hd)
        copies = int(min(256, max(2, -(-COLD_BYTES // (ctx * n_kv * hd * 8)))))
        for mode in ("exact", "fast"):
            iters = max(8, copies) if ctx <= 4096 else 8
            hip.bench_attention(heads, kv_mul, hd, ctx, 1, 2, args.seed, mode)
            hip.profile_enable(True)
            o = hip.bench_attention(heads, kv_mul, hd, ctx, copies, iters, args.seed, mode)
            prof = hip.profile_results()
            hip.profile_enable(False)
            parts = {f: prof[f][0] / prof[f][1] * 1e3 for f in fams[mode] if f in prof and prof[f][1]}
            if any(f not in parts for f in fams[mode] if f not in optional) or not np.all(np.isfinite(o)):
                raise SystemExit(f"sweep attention {mode} ctx {ctx}: missing launches or non-finite output")
            us = sum(parts.values())
            gbs = alg / (us * 1e-6) / 1e9
            attn.append({"mode": mode, "ctx": ctx, "heads": [heads, n_kv], "head_dim": hd, "alg_bytes": alg,
                         "us_per_call": round(us, 3), "kernel_us": {k: round(v, 3) for k, v in parts.items()},
                         "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "copies": copies})
            log(f"attention {mode:5s} ctx {ctx:6d}: {us:9.2f} us  {gbs:7.1f} GB/s  frac {gbs / HBM_PEAK_GBS:.3f}  "
                + " ".join(f"{k}={v:.1f}" for k, v in parts.items()))
    print(json.dumps({"sweep": {"peak_GBps": HBM_PEAK_GBS, "gemv": gemv, "attention": attn,
                                "workload": "BASELINE configs[1]: batch-1 GEMV per format/shape, GQA decode "
                                            "attention 32q/8kv/128 (pseudo-normal K/V, linear slots)"}}),
          flush=True)


def recorded_traffic(args, path=TRAFFIC_FILE):
    """HBM bytes per launch of a roofline kernel, from the two rocprofv3
    --pmc passes (FETCH_SIZE, WRITE_SIZE) recorded for this workload, each
    scaled by the same counter's reading on a copy kernel of known size."""
    if args.config != "llama3-8b-q4km" or args.ctx != 4096 or not os.path.exists(path):
        return None
    with open(path) as f:
        rec = json.load(f)
    return rec.get("traffic_bytes_per_launch")


def copy_probe(mib):
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, dtype=torch.float32, device="cuda")
    y = torch.empty_like(x)
    for _ in range(5):
        torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    log(f"copy probe: 5 x {mib} MiB read + {mib} MiB written")


def cpu_baseline(model, res, storage, args, log):
    """The CPU oracle (oracle/, a C restatement of the reference's x86 AVX2
    path with its 64-row dynamic worker split) continues the decode from the
    GPU's KV cache: same weights, same context length, bounded sample."""
    import numpy as np
    from oracle import oracle as O

    cfg = model["config"]
    cores = host_cores()
    t0 = time.time()
    orc = O.OracleModel(model, storage_len=storage, threads=cores)
    # next position to decode (the last greedy step left pos here)
    pos0 = args.ctx + args.warmup + args.steps + args.profile_tokens - 1
    for layer in range(cfg["n_layers"]):
        ok, ov = orc.kv(layer, storage)
        w = cfg["n_kv_heads"] * cfg["head_dim"]
        ok[: pos0 * w] = res.kv_read(layer, 0, 0, pos0)
        ov[: pos0 * w] = res.kv_read(layer, 1, 0, pos0)
    log(f"cpu baseline: KV copied in {time.time() - t0:.1f}s, {cores} threads")
    tok = 1
    n = 0
    t_start = time.time()
    pos = pos0
    while pos < storage and (n < 2 or time.time() - t_start < args.cpu_seconds):
        logits = orc.forward(tok, pos)
        tok, _ = O.greedy(logits, [], 1.0)
        pos += 1
        n += 1
    dt = time.time() - t_start
    v = n / dt
    log(f"cpu baseline: {n} tokens in {dt:.1f}s -> {v:.2f} tok/s")
    return {"value": round(v, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"{n} greedy decode tokens of the same model at ctx {pos0}..{pos0 + n} "
                      f"(C restatement of the reference AVX2 path, {cores} threads)"}


if __name__ == "__main__":
    main()
