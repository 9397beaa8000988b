#!/usr/bin/env python3
"""Batch-1 decode benchmark on one MI355X.

Workload (default): the Qwen3-0.6B-shaped Q4_K_M decoder (hidden 1024, 28
layers, 16 q / 8 kv heads, head_dim 128, FFN 3072, vocab 151936, tied Q6_K
lm_head), random N(0, 0.02) weights, a 2048-token seeded random prompt
prefilled on the device, then greedy decode with an fp16 K/V cache. A step is
one decode token; `value` is decode tokens/s over the K timed steps (weights
and K/V cache resident in HBM; timed with HIP events on the engine stream).

Also reported:
  roofline      the kernel class with the most time per step, its algorithmic
                bytes per launch / mean launch time (every layer's launch of the
                class back to back, HIP events) vs 8 TB/s;
  step_roofline weight + K/V bytes per token / ms per token vs 8 TB/s;
  q4k_matvec    the Q4_K gate|up matvec's GB/s;
  cpu_baseline  the oracle (CPU restatement of the reference WGSL
                arithmetic) timed on a bounded sample of the same decode;
  prefill_*     the prompt pass (row batches on the matrix cores);
  batched_decode 64 sequences x 512-token prompts, greedy steps over all of
                them at once (the batched configuration).
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "batch-1 decode tokens/s + Q4_K matvec achieved GB/s vs HBM peak, 1×MI355X"
HBM_PEAK_GBS = 8000.0


def kernel_class(name: str) -> str:
    return name.split(".", 1)[1] if "." in name else name


def build_model(workload: str, cache_dir: Path) -> str:
    from chonklm_amd import write_synthetic_gguf

    cache_dir.mkdir(parents=True, exist_ok=True)
    path = cache_dir / f"{workload}.gguf"
    if not path.exists():
        tmp = cache_dir / f"{workload}.gguf.tmp"
        write_synthetic_gguf(workload, str(tmp), threads=min(16, os.cpu_count() or 4))
        os.replace(tmp, path)
    return str(path)


def profiled_traffic(kernel: str, workload: str):
    """HBM bytes per launch of `kernel` on `workload` from the rocprofv3 FETCH_SIZE /
    WRITE_SIZE summaries kept under profiles/ (lines 'traffic: <kernel> <workload> <bytes>')."""
    for f in sorted((ROOT / "profiles").glob("*.md")):
        for line in f.read_text().splitlines():
            if line.startswith("traffic: "):
                rest = line[len("traffic: "):].rsplit(" ", 2)
                if len(rest) == 3 and rest[0] == kernel and rest[1] == workload:
                    return int(rest[2])
    return None


def kernel_symbol(cls: str, info: dict) -> str:
    """Kernel function behind a step's kernel class (as rocprofv3 names it)."""
    g = info["heads"] // info["kv_heads"]
    hd = info["head_dim"]
    kv16 = "true" if info.get("kv_dtype", 0) == 0 else "false"  # CHONK_KV_F16 == 0
    # the engine's rule for the register-resident decode attention (attn_dec_supported)
    dec = (kv16 == "true" and hd in (64, 128, 256) and 1 <= g <= 8 and g * hd <= 1536
           and (info["context"] + 63) // 64 <= 128 * 16 and os.environ.get("CHONK_ATTN") != "chunked")
    walk = "true" if (info["context"] + 63) // 64 > 128 else "false"  # sub-chunks per workgroup (long contexts)
    attn = f"k_attn_dec<{g}, {hd}, {walk}>" if dec else f"k_attention<{g}, {kv16}>"
    if os.environ.get("CHONK_MV") == "generic":
        mv = {"gateup": "k_mv_swiglu", "qkv": "k_mv_store", "oproj": "k_mv_add", "down": "k_mv_add"}
    elif info.get("architecture") == 3:  # gpt2 row kernels (LayerNorm prologues, biases)
        mv = {"gateup": "k_mvr_gelu_ln", "qkv": "k_mvr_store_ln", "oproj": "k_mvr_add_bias", "down": "k_mvr_add_bias"}
    else:  # one-row-per-lane-group kernels (layers after the first; llama/qwen3 prologues)
        mv = {"gateup": "k_mvr_swiglu_norm", "qkv": "k_mvr_store_norm", "oproj": "k_mvr_add_plain",
              "down": "k_mvr_add_plain", "inproj": "k_mvr_store_norm", "outproj": "k_mvr_add_conv",
              "ssm": "k_mamba_ssm"}
        if info.get("architecture") == 6:  # granitehybrid: out_proj's prologue is the gated norm
            mv["outproj"] = "k_mvr_add_gate"
    if info["ffn"] > 4096 and "down" in mv and os.environ.get("CHONK_MV") != "generic":
        mv["down"] = "k_mvr_add_bias_wide"  # rows above 4096 stage the input through LDS
    # the q|k|v matvec and the decode attention in one launch (layers after the first)
    fused = f"k_qkv_attn<{g}, {hd}>"
    return {"attn": attn, "qkv_attn": fused, "lmhead": "k_mv_logits", **mv}.get(cls, cls)


def host_cpus() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(path: str, w, pos: int, seconds: float, threads: int) -> dict:
    """Oracle decode steps at the benchmark's context (fake K/V, greedy), plus a few
    prompt steps without logits at two contexts, from which the reference's own figure
    generated / (prefill + decode) (llama-wgsl-runtime.ts:266, :312-313) is estimated
    for the whole workload (per-token cost taken as linear in the position)."""
    from oracle.oracle import OracleModel

    ctx = max(pos + 64, w.prompt_tokens + w.decode_tokens + 8)
    ref = OracleModel(path, w.spec.vocab, w.spec.layers, ctx, kv_f16=True, threads=threads)
    ref.fake_context(pos, seed=1)
    tok = 1
    n = 0
    t0 = time.perf_counter()
    while True:
        tok = ref.run_token(tok, True)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 64:
            break
    decode_s = el / n
    # prompt steps (runToken(id, false): no lm_head) at the start and in the middle of the prompt
    samples = []
    for p0 in (0, w.prompt_tokens // 2):
        ref.reset()
        ref.fake_context(p0, seed=2)
        t1 = time.perf_counter()
        for i in range(4):
            ref.run_token(1 + i, False)
        samples.append((p0 + 2, (time.perf_counter() - t1) / 4))
    ref.close()
    (x0, c0), (x1, c1) = samples
    slope = (c1 - c0) / max(x1 - x0, 1)
    prefill_est = sum(max(c0 + slope * (p - x0), 0.0) for p in range(w.prompt_tokens - 1))
    decode_est = w.decode_tokens * decode_s
    return {"value": n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
            "host_cpus": host_cpus(),
            "reference_formula_tokens_per_sec": round(w.decode_tokens / (prefill_est + decode_est), 4),
            "reference_formula_note": f"generated / (prefill + decode) for {w.prompt_tokens} prompt + "
                                      f"{w.decode_tokens} generated tokens, estimated from the sampled per-token "
                                      f"costs (prompt steps {c0 * 1e3:.0f} ms at position {x0}, {c1 * 1e3:.0f} ms at "
                                      f"{x1}; decode {decode_s * 1e3:.0f} ms at {pos})",
            "sample": f"{n} greedy decode steps of the same model at context {pos}..{pos + n} "
                      f"(synthetic K/V) and 8 prompt steps, oracle CPU restatement of the reference WGSL "
                      f"arithmetic on {threads} threads ({host_cpus()} host CPUs visible), {el:.1f} s of decode"}


def kernel_cold_warm(eng, info: dict, reps: int) -> dict:
    """Per-launch HIP-event times of representative step kernels with the caches flushed
    (cold: >= 512 MiB written first, evicting L2 and the 256 MB Infinity Cache) and right
    after an identical launch (warm), each over `reps` launches, with their GB/s."""
    n = info["kernels_per_step"]
    names = {}
    for kid in range(n - 1):
        name, _, nbytes = eng.bench_kernel(kid, 1)
        names[name] = (kid, nbytes)
    last = info["layers"] - 1
    want = {"attn (last layer)": f"L{last}.attn", "gate|up Q4_K (layer 1)": "L1.gateup",
            "q|k|v (layer 1)": "L1.qkv", "down (layer 1)": "L1.down", "lm_head": "lmhead"}
    out = {}
    for label, key in want.items():
        if key not in names:
            continue
        kid, nbytes = names[key]
        cold, warm = eng.bench_kernel_cold(kid, reps)
        out[label] = {"kernel": key, "bytes": int(nbytes), "cold_us": round(cold, 3), "warm_us": round(warm, 3),
                      "cold_gb_s": round(nbytes / cold / 1e3, 1), "warm_gb_s": round(nbytes / warm / 1e3, 1)}
    return out


def q4k_matvec_bandwidth(rows: int = 262144, k: int = 2048, reps: int = 20) -> dict:
    """A Q4_K matvec too large for the Infinity Cache (rows x k Q4_K = 302 MB): every launch
    streams the matrix from HBM; GB/s of its GGUF bytes over the mean of `reps` launches."""
    import ctypes as C

    from chonklm_amd._lib import check, lib

    nb = rows * (k // 256)
    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    blocks[:, 0:4] = np.array([0x00, 0x20, 0x00, 0x20], dtype=np.uint8)  # d = dmin = 2^-7 (f16)
    x = rng.standard_normal(k).astype(np.float32)
    y = np.empty(rows, dtype=np.float32)
    us = C.c_double()
    check(lib().chonk_matvec(0, 12, blocks.ctypes.data, rows, k, x.ctypes.data_as(C.POINTER(C.c_float)),
                             y.ctypes.data_as(C.POINTER(C.c_float)), reps, C.byref(us)))
    nbytes = nb * 144
    return {"rows": rows, "k": k, "bytes": nbytes, "us_per_launch": round(us.value, 2),
            "achieved": round(nbytes / us.value / 1e3, 1), "unit": "GB/s",
            "frac": round(nbytes / us.value / 1e3 / HBM_PEAK_GBS, 4),
            "note": "generic Q4_K matvec kernel, 256-row tiles; matrix larger than the Infinity Cache"}


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16


def gemm_params(spec) -> int:
    """Weights of every linear layer of a step (q, k, v, o, gate, up, down per
    layer and the lm_head): a decode batch multiplies each by every row."""
    hd = spec.head_dim or spec.hidden // spec.heads
    per_layer = spec.hidden * (spec.heads + 2 * spec.kv_heads) * hd + spec.heads * hd * spec.hidden \
        + 3 * spec.hidden * spec.ffn
    return spec.layers * per_layer + spec.hidden * spec.vocab


def batched_decode(eng, vocab: int, seqs: int, prompt: int, steps: int, warmup: int, spec=None) -> dict:
    """The batched-decode configuration: `seqs` independent sequences with a
    `prompt`-token random prompt each, then greedy steps over all of them at
    once (one MFMA GEMM per linear layer over the batch rows, paged fp16 K/V)."""
    from chonklm_amd.runtime import LlamaWgslBatch

    b = LlamaWgslBatch(eng, seqs, prompt + warmup + steps + 1)
    rng = np.random.default_rng(7)
    t0 = time.perf_counter()
    cur = [b.prefill(s, rng.integers(0, vocab, prompt).tolist()) for s in range(seqs)]
    prefill_s = time.perf_counter() - t0
    rows = list(range(seqs))
    for _ in range(warmup):
        cur = b.step(rows, cur)
    t1 = time.perf_counter()
    for _ in range(steps):
        cur = b.step(rows, cur)
    el = time.perf_counter() - t1
    b.close()
    out = {"sequences": seqs, "prompt_tokens": prompt, "steps": steps, "warmup": warmup,
           "ms_per_step": round(1000.0 * el / steps, 4) if steps else None,
           "tokens_per_sec": round(seqs * steps / el, 1) if steps else None,
           "prefill_tokens_per_sec": round(seqs * prompt / prefill_s, 1),
           "note": "host-timed, step = one greedy token for every sequence"}
    if spec is not None and steps:
        # matrix-core use of the whole step: the GEMMs' algorithmic flops (2 x rows x
        # weights) and the products the hi/lo fp16 split issues (3 per weight-row pair)
        alg = 2.0 * seqs * gemm_params(spec) / (el / steps) / 1e12
        out["mfma_util"] = {"alg_tflops": round(alg, 2), "issued_tflops": round(3 * alg, 2),
                            "peak_tflops": MFMA_PEAK_TFLOPS, "frac_alg": round(alg / MFMA_PEAK_TFLOPS, 4),
                            "frac_issued": round(3 * alg / MFMA_PEAK_TFLOPS, 4),
                            "note": "step-level: GEMM flops over the whole step time (attention and glue "
                                    "included); the per-kernel counters are in profiles/"}
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", default="qwen3-0.6b-q4_k_m")
    ap.add_argument("--kv-dtype", default="f16", choices=["f16", "f32"],
                    help="K/V cache element type (the reference keeps fp32 K/V)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kernel-rounds", type=int, default=10,
                    help="back-to-back passes over each kernel class (one launch per layer) timed with HIP events")
    ap.add_argument("--cold-reps", type=int, default=100,
                    help="launches per kernel for the cold / warm per-launch timing (0 skips it)")
    ap.add_argument("--no-kernel-times", action="store_true",
                    help="skip the per-kernel timing pass (profiling runs)")
    ap.add_argument("--fake-prefill", action="store_true",
                    help="fill the K/V cache with synthetic values instead of prefilling the prompt "
                         "(profiling runs: the trace then holds decode steps only)")
    ap.add_argument("--model-cache", default=os.environ.get("CHONK_MODEL_CACHE", "/tmp/chonk_models"))
    ap.add_argument("--no-batched", action="store_true", help="skip the batched-decode measurement")
    ap.add_argument("--batched-only", action="store_true",
                    help="only the batched-decode measurement (profiling runs: per-step kernel time is the "
                         "difference of two runs with different --batched-steps)")
    ap.add_argument("--batched-steps", type=int, default=32)
    ap.add_argument("--prompt-tokens", type=int, default=0,
                    help="override the workload's prompt length (with --fake-prefill the K/V rows are filled "
                         "synthetically): contexts past 8192 positions run the chunked decode attention")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first run 4 device-to-device copies of MIB MiB (a known-size kernel for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1:
        print("bench.py measures one GPU: batch-1 decode does not shard across GPUs "
              "(see DESIGN.md, 'More than one GPU'); run with --gpus 1", file=sys.stderr)
        return 2

    from chonklm_amd import (WORKLOADS, generate_llama_wgsl, load_gpt_wgsl_model, load_granite_wgsl_model,
                             load_lfm_wgsl_model,
                             load_llama_wgsl_model)

    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy << 20
        src = torch.ones(n, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(f"calibration: 4 copies of {n} bytes", file=sys.stderr)
        del src, dst

    w = WORKLOADS[args.workload]
    if args.prompt_tokens > 0:
        w = dataclasses.replace(w, prompt_tokens=args.prompt_tokens)
    t_build = time.perf_counter()
    path = build_model(args.workload, Path(args.model_cache))
    build_s = time.perf_counter() - t_build

    ctx = w.prompt_tokens + 1 + args.warmup + args.steps + 8
    md = w.model_def(path, kv_dtype=args.kv_dtype)
    md.max_context = ctx
    loaded = {"gpt-webgpu": load_gpt_wgsl_model, "lfm2-webgpu": load_lfm_wgsl_model,
              "granite-webgpu": load_granite_wgsl_model}.get(
        md.runtime, load_llama_wgsl_model)(md)
    eng = loaded.engine
    info = eng.info
    prompt = w.prompt(1234)

    if args.batched_only:
        bd = batched_decode(eng, w.spec.vocab, 64, 512, args.batched_steps, 4, w.spec)
        print(json.dumps({"metric": "batched decode tokens/s (64 sequences), 1xMI355X", "batched_decode": bd,
                          "config": {"workload": w.name}}))
        eng.dispose()
        return 0

    if args.fake_prefill:
        eng.fake_context(w.prompt_tokens, seed=1)
        eng.run_token(prompt[-1], True)
        prefill_ms = float("nan")
    else:
        # device prefill of the prompt (+ the first generated token)
        out = generate_llama_wgsl(loaded, prompt, 1)
        prefill_ms = out["prefillMs"]
    pos0 = eng.position

    # timed greedy decode
    t0 = time.perf_counter()
    ms = eng.bench_decode(args.warmup, args.steps)
    wall_ms = (time.perf_counter() - t0) * 1000.0
    ms_per_step = ms / args.steps
    tok_s = 1000.0 / ms_per_step
    pos_end = eng.position

    # per-launch durations (HIP events on the engine stream): each kernel class (one
    # launch per layer, e.g. every layer's attention) launched back to back, so every
    # launch meets its weights / K/V rows as cold as in the step; bytes at this position
    n_kernels = info["kernels_per_step"]
    classes: dict[str, dict] = {}
    if not args.no_kernel_times:
        ids_of: dict[str, list[int]] = {}
        for kid in range(n_kernels - 1):  # the select kernel moves no bulk data
            name, _, nbytes = eng.bench_kernel(kid, 0)
            ids_of.setdefault(kernel_class(name), []).append(kid)
            c = classes.setdefault(kernel_class(name), {"launches": 0, "us": 0.0, "bytes": 0})
            c["launches"] += 1
            c["bytes"] += nbytes
        for cls, ids in ids_of.items():
            classes[cls]["us"] = eng.time_kernels(ids, args.kernel_rounds) * len(ids)
    if not classes:
        classes["none"] = {"launches": 1, "us": float("nan"), "bytes": 0}
    gu = classes.get("gateup")

    # whole-step bytes: weights + K/V read at the mean timed position + K/V write
    kvdim = info["kv_heads"] * info["head_dim"]
    mean_pos = (pos0 + args.warmup + pos_end) / 2.0
    kv_elem = 2 if info.get("kv_dtype", 0) == 0 else 4
    # (lfm2: only the attention layers hold a K/V cache)
    kv_layers = sum(1 for k in (w.spec.layer_kv_heads or [1] * info["layers"]) if k > 0)
    kv_bytes = 2 * kv_layers * kvdim * (mean_pos + 1) * kv_elem
    step_bytes = info["weight_bytes_per_token"] + kv_bytes
    step_gbs = step_bytes / (ms_per_step * 1e-3) / 1e9

    dom_name, dom = max(classes.items(), key=lambda kv: kv[1]["us"])
    dom_us = dom["us"] / dom["launches"]
    dom_bytes = dom["bytes"] / dom["launches"]
    dom_gbs = dom_bytes / dom_us / 1e3

    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": w.description or w.name,
            "name": w.name,
            "batch": 1,
            "prompt_tokens": w.prompt_tokens,
            "context_at_timed_start": pos0 + args.warmup,
            "context_at_end": pos_end,
            "kv_cache": "f16" if info.get("kv_dtype", 0) == 0 else "f32",
            "weights": f"{w.spec.recipe.upper()} GGUF (llama.cpp type recipe), random N(0,0.02)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dom_name,
            "achieved": round(dom_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom_gbs / HBM_PEAK_GBS, 4),
            "traffic": profiled_traffic(kernel_symbol(dom_name, info), w.name),
            "kernel_symbol": kernel_symbol(dom_name, info),
            "bytes_per_launch": int(dom_bytes),
            "us_per_launch": round(dom_us, 3),
        },
        "step_roofline": {
            "bytes_per_token": int(step_bytes),
            "weight_bytes_per_token": int(info["weight_bytes_per_token"]),
            "achieved": round(step_gbs, 1),
            "unit": "GB/s",
            "frac": round(step_gbs / HBM_PEAK_GBS, 4),
        },
        "q4k_matvec": None if not gu else {
            "kernel": "gateup (Q4_K, fused RMSNorm + SwiGLU)",
            "achieved": round(gu["bytes"] / gu["us"] / 1e3, 1), "unit": "GB/s",
            "us_per_launch": round(gu["us"] / gu["launches"], 3)},
        # per-step time of each kernel class (HIP events over back-to-back passes of the class)
        "kernels": {k: {"launches": v["launches"], "us_per_step": round(v["us"], 2),
                        "gb_s": round(v["bytes"] / v["us"] / 1e3, 1)} for k, v in classes.items()},
        "kernel_sum_us": round(sum(v["us"] for v in classes.values()), 2),
        "wall_ms_timed": round(wall_ms, 3),
        "prefill_ms": None if prefill_ms != prefill_ms else round(prefill_ms, 2),
        "prefill_tokens_per_sec": None if prefill_ms != prefill_ms else round(w.prompt_tokens / (prefill_ms / 1000.0), 1),
        "model_build_s": round(build_s, 1),
        "cpu_baseline": None,
    }
    if w.temperature > 0 or w.top_k > 0:
        # the timed steps above select greedily; the configuration's own sampling runs
        # through the device-driven generate loop (candidate sampler in the select kernel)
        from chonklm_amd.runtime import reset_llama_wgsl_conversation

        reset_llama_wgsl_conversation(loaded)
        g = generate_llama_wgsl(loaded, prompt, w.decode_tokens, temperature=w.temperature, top_k=w.top_k,
                                top_p=w.top_p, seed=9)
        n_gen = len(g["ids"])
        result["sampled_decode"] = {
            "temperature": w.temperature, "top_k": w.top_k, "generated": n_gen,
            "tokens_per_sec": round((n_gen - 1) / (g["decodeMs"] / 1000.0), 1) if n_gen > 1 else None,
            "note": "generateLlamaWgsl with the configuration's sampling; decode wall time after the prompt"}
    if args.cold_reps > 0 and not args.no_kernel_times:
        result["kernel_cold_warm"] = kernel_cold_warm(eng, info, args.cold_reps)
        result["q4k_matvec_hbm"] = q4k_matvec_bandwidth()
    if not args.no_batched and info.get("kv_dtype", 0) == 0 and info.get("architecture") not in (3, 5):
        result["batched_decode"] = batched_decode(eng, w.spec.vocab, 64, 512, 32, 4, w.spec)
    if not args.no_cpu_baseline:
        threads = min(16, host_cpus())  # the GPU box's CPU share is 16 threads
        result["cpu_baseline"] = cpu_baseline(path, w, pos0, args.cpu_seconds, threads)
    loaded.engine.dispose()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
